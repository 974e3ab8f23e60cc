"""Speculative-decoding engine over the device-resident verification round.

Drop-in for src/myvllm/spec_engine/spec_llm_engine.py (and the LLMEngine
surface it inherits, engine/llm_engine.py:26-143):

  * configuration keys (:32-102): ``spec_method`` ("ngram", "model",
    "hybrid", or "none" for plain decoding through the same round),
    ``num_speculative_tokens``, ``ngram_min_size``, ``ngram_max_size``,
    ``max_num_sequences``, ``max_num_batched_tokens``, ``max_model_length``,
    ``block_size``, ``eos``, ``world_size`` (must be 1, :34-35),
    ``enforce_eager`` / ``capture_verify``;
  * ``add_token_ids`` (llm_engine.py:84-87), ``generate_token_ids(prompts,
    params)`` (:138-143) and ``generate`` (token-id prompts: no tokenizer is
    loaded here), returning the reference's result dict: ``token_ids`` per
    request in request order, and ``metrics`` with ``total_s``, ``ttft_s``,
    ``prefill_tokens``, ``decode_tokens``, ``output_tokens``,
    ``prefix_cache`` (:118-132) and ``spec_decoding`` (:305-312: ``rounds``,
    ``drafted_tokens``, ``accepted_tokens``, ``fallback_rounds``, cumulative
    over calls, plus ``model_fallback_rounds`` / ``model_fallback_seqs`` for
    a hybrid drafter);
  * ``pin_prefix(token_ids)`` (:145-146), ``exit()`` (:294-303) and the
    context-manager protocol (:148-152).

The target is a random-init Qwen3 of the shape in ``config["model_config"]``
(Qwen3-0.6B by default); the model / hybrid drafter a random-init Qwen3 of
``config["draft_model_config"]`` that shares the target's vocabulary,
pages and block tables (no checkpoint loading: the reference fetches
weights by name, which this build does not do).

Scheduling (engine/scheduler.py): requests wait in the scheduler's queue;
whenever round slots are free, waiting requests are admitted in order
while the token budget (prompt tokens not served by the prefix cache) and
the free pages allow, each with pages for its whole life (prompt +
max_tokens + K + 1 positions) so the device round never waits for the
host; the admitted batch is prefilled in one forward (the pages its prefix
cache covers are skipped), then every slot advances through the captured
round until it finishes, and its slot takes the next waiting request.

Sampling: a request with temperature <= 1e-6 is decoded greedily; any
other temperature samples the first token, the model drafts and the
acceptance (min(1, p_t/p_d) with residual resampling) from torch's device
generator, seeded from ``config["seed"]``.
"""

from __future__ import annotations

import atexit
import math
import time
import weakref

import torch

from naivllm_amd.engine.scheduler import Scheduler
from naivllm_amd.engine.sequence import Sequence, SequenceStatus
from naivllm_amd.engine.verify_round import VerifyRound
from naivllm_amd.layers.qwen3 import Qwen3Config, Qwen3Verify
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine.rejection_sampler import GREEDY_TEMPERATURE, sample


def _exit_if_alive(ref) -> None:
    engine = ref()
    if engine is not None:
        engine.exit()


class SpecLLMEngine:
    def __init__(self, config: dict):
        assert config.get("world_size", 1) == 1, "speculative decoding currently supports world_size == 1"
        self.spec_method = config.get("spec_method", "ngram")
        if self.spec_method not in ("ngram", "model", "hybrid", "none"):
            raise ValueError(f"spec_method {self.spec_method!r}: expected 'ngram', 'model', 'hybrid' or 'none'")
        self.num_speculative_tokens = config.get("num_speculative_tokens", 5)
        self.min_ngram = config.get("ngram_min_size", 2)
        self.max_ngram = config.get("ngram_max_size", 8)
        self.max_num_sequences = config.get("max_num_sequences", 8)
        self.max_num_batched_tokens = config.get("max_num_batched_tokens", 16384)
        self.max_model_length = config.get("max_model_length", 4096)
        self.block_size = config.get("block_size", 256)
        self.eos = config.get("eos_token_id", config.get("eos", -1))
        self.device = torch.device(config.get("device", "cuda"))
        seed = config.get("seed", 0)
        torch.manual_seed(seed)  # the device generator of the sampled draws
        cfg = config.get("model_config") or Qwen3Config()
        self.model = Qwen3Verify(cfg, self.device, seed=seed)
        self.draft_model = None
        if self.spec_method in ("model", "hybrid"):
            dcfg = config.get("draft_model_config") or Qwen3Config.qwen3_0_6b()
            if dcfg.vocab_size != cfg.vocab_size:
                raise ValueError("draft and target models must share the tokenizer/vocabulary")
            self.draft_model = Qwen3Verify(dcfg, self.device, seed=config.get("draft_seed", seed + 1))
            self.draft_model.decode_linears = True  # its one- and two-row steps
        K = self.num_speculative_tokens
        self.history_len = self.max_model_length + K + 1
        self.max_blocks = math.ceil(self.history_len / self.block_size)
        num_blocks = config.get("num_kvcache_blocks", self.max_num_sequences * self.max_blocks)
        self.scheduler = Scheduler(self.max_num_sequences, self.max_num_batched_tokens, num_blocks, self.block_size,
                                   self.eos)
        self.block_manager = self.scheduler.block_manager
        self.model.allocate_kv_cache(num_blocks, self.block_size)
        if self.draft_model is not None:
            self.draft_model.allocate_kv_cache(num_blocks, self.block_size)
        self.eager = config.get("enforce_eager", False) or not config.get("capture_verify", True)
        self.rounds: dict[bool, VerifyRound] = {}  # greedy / stochastic round, built on first use
        self.spec_stats = {"method": self.spec_method, "num_speculative_tokens": K, "rounds": 0,
                           "drafted_tokens": 0, "accepted_tokens": 0, "fallback_rounds": 0}
        if self.spec_method == "hybrid":
            self.spec_stats.update(model_fallback_rounds=0, model_fallback_seqs=0)
        self._closed = False
        # exit() at interpreter exit, through a weak reference so that the
        # registration does not keep a deleted engine (and its caches) alive
        atexit.register(_exit_if_alive, weakref.ref(self))

    # -------------------------------------------------------------- lifecycle
    def exit(self) -> None:
        """Release the captured rounds and the KV caches (llm_engine.py:52-59);
        idempotent, also run at interpreter exit."""
        if self._closed:
            return
        self._closed = True
        self.rounds.clear()
        for m in (self.model, self.draft_model):
            if m is not None:
                m.k_caches, m.v_caches = [], []
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc_value, traceback):
        self.exit()

    def _check_open(self) -> None:
        if self._closed:
            raise RuntimeError("the engine was closed by exit()")

    # ---------------------------------------------------------------- rounds
    @property
    def round(self) -> VerifyRound:
        """The greedy round."""
        return self._round(False)

    def _round(self, stochastic: bool) -> VerifyRound:
        """The greedy or the stochastic round, built and captured on first use."""
        r = self.rounds.get(stochastic)
        if r is None:
            r = VerifyRound(self.model, self.max_num_sequences, self.num_speculative_tokens, self.min_ngram,
                            self.max_ngram, self.history_len, self.max_blocks, self.eos, method=self.spec_method,
                            draft_model=self.draft_model, stochastic=stochastic)
            if not self.eager:
                r.capture()
            self.rounds[stochastic] = r
        return r

    # ---------------------------------------------------------------- prefill
    @torch.inference_mode()
    def _prefill(self, seqs: list[Sequence]) -> list[int]:
        """One forward over the new prompt tokens of ``seqs`` (each from its
        first page the prefix cache does not serve), mirrored into the draft
        model's cache when there is one (spec_llm_engine.py:147-151); returns
        each sequence's first completion token, sampled from its last prompt
        row as the reference's prefill + sampler (layers/sampler.py:14-24) do."""
        toks = [s.token_ids for s in seqs]
        starts = [s.num_cached_tokens for s in seqs]
        tables = [s.block_table for s in seqs]
        logits = self.model.prefill(toks, starts, tables)
        if self.draft_model is not None:
            self.draft_model.prefill(toks, starts, tables)
        temps = torch.tensor([float(s.temperature) for s in seqs], dtype=torch.float32, device=self.device)
        if all(s.temperature <= GREEDY_TEMPERATURE for s in seqs):
            return logits.argmax(-1).tolist()
        noise = torch.empty(len(seqs), logits.shape[-1], dtype=torch.float32,
                            device=self.device).exponential_(1).clamp_min_(1e-10)
        return sample(logits, temps, noise).tolist()

    def _load_slot(self, r: VerifyRound, slot: int, seq: Sequence) -> None:
        """Write a prefilled sequence's state into round slot ``slot``."""
        dev = self.device
        r.history[slot, :seq.num_tokens] = torch.tensor(seq.token_ids, dtype=torch.int32, device=dev)
        r.hist_len[slot] = seq.num_tokens
        r.prompt_len[slot] = seq.num_prompt_tokens
        r.max_tokens[slot] = seq.max_tokens
        r.max_len[slot] = seq.max_model_length or self.max_model_length
        r.ignore_eos[slot] = int(seq.ignore_eos)
        r.temperature[slot] = float(seq.temperature)
        r.block_tables[slot].fill_(-1)
        r.block_tables[slot, :len(seq.block_table)] = torch.tensor(seq.block_table, dtype=torch.int32, device=dev)
        r.active[slot] = 1

    def _cap(self, seq: Sequence) -> int:
        """Tokens the sequence may reach: prompt + max_tokens within its and
        the engine's length limits."""
        return min(seq.num_prompt_tokens + seq.max_tokens, seq.max_model_length or self.max_model_length,
                   self.max_model_length)

    # ------------------------------------------------------------- requests
    def add_token_ids(self, token_ids: list[int], sampling_params: SamplingParams) -> int:
        self._check_open()
        if isinstance(token_ids, str):
            raise ValueError("prompts are token-id lists: this build loads no tokenizer")
        seq = Sequence(list(token_ids), sampling_params)
        if not seq.token_ids:
            raise ValueError("empty prompt")
        if len(seq.token_ids) >= self.history_len - self.num_speculative_tokens - 1:
            raise ValueError("prompt longer than max_model_length")
        self.scheduler.add_sequence(seq)
        return seq.seq_id

    def pin_prefix(self, token_ids: list[int]) -> int:
        """Keep the cached full pages of ``token_ids`` resident (a prefix
        evaluated by an earlier request); returns the tokens they cover."""
        return self.block_manager.pin_prefix(list(token_ids))

    def unpin_all(self) -> None:
        self.block_manager.unpin_all()

    def generate_token_ids(self, prompts: list[list[int]], sampling_params: SamplingParams | list[SamplingParams]
                           ) -> dict:
        """Generate from pre-tokenised prompts (llm_engine.py:138-143)."""
        params = sampling_params if isinstance(sampling_params, list) else [sampling_params] * len(prompts)
        if len(params) != len(prompts):
            raise ValueError("one SamplingParams per prompt")
        waiting = list(self.scheduler.waiting)
        ids = [self.add_token_ids(p, sp) for p, sp in zip(prompts, params)]
        seqs = [s for s in self.scheduler.waiting if s.seq_id in set(ids)]
        assert len(seqs) == len(ids) and len(waiting) + len(ids) == len(self.scheduler.waiting)
        return self._generate(seqs)

    def generate(self, prompts: list[list[int]], sampling_params: SamplingParams | list[SamplingParams]) -> dict:
        """generate_token_ids (prompts are token-id lists)."""
        return self.generate_token_ids(prompts, sampling_params)

    # --------------------------------------------------------------- the loop
    @torch.inference_mode()
    def _generate(self, requests: list[Sequence]) -> dict:
        self._check_open()
        K = self.num_speculative_tokens
        r = self._round(any(s.temperature > GREEDY_TEMPERATURE for s in self.scheduler.waiting))
        slots: list[Sequence | None] = [None] * r.max_batch
        left: dict[int, int] = {}  # slot -> tokens its sequence may still commit
        t0 = time.perf_counter()
        first_token_t = None
        prefill_s = 0.0
        prefill_tokens = decode_tokens = rounds = 0
        pending = None  # (bucket, report slot) of a launched round whose report is unread
        rep_slot = 0

        def finish(i: int) -> None:
            seq = slots[i]
            n = int(r.hist_len[i])
            seq.token_ids = r.history[i, :n].tolist()
            seq.num_tokens = n
            seq.last_token = seq.token_ids[-1]
            self.block_manager.register_full_pages(seq)
            self.scheduler.finish(seq)
            r.active[i] = 0
            r.hist_len[i] = 0
            slots[i] = None
            left.pop(i, None)

        while self.scheduler.waiting or any(s is not None for s in slots) or pending is not None:
            free = [i for i, s in enumerate(slots) if s is None]
            if self.scheduler.waiting and free and pending is None:
                tp = time.perf_counter()
                batch = self.scheduler.admit(len(free), reserve=lambda s: self._cap(s) + K + 1)
                if batch:
                    prefill_tokens += sum(s.num_tokens - s.num_cached_tokens for s in batch)
                    firsts = self._prefill(batch)
                    for seq, tok, i in zip(batch, firsts, free):
                        seq.append_token(tok)
                        slots[i] = seq
                        self._load_slot(r, i, seq)
                        left[i] = self._cap(seq) - seq.num_tokens
                        if left[i] <= 0 or (not seq.ignore_eos and tok == self.eos):
                            finish(i)
                    torch.cuda.synchronize(self.device)
                    now = time.perf_counter()
                    prefill_s += now - tp
                    if first_token_t is None:
                        first_token_t = now
                elif not any(s is not None for s in slots):
                    raise RuntimeError("no request can be admitted: not enough free KV pages for its reservation")
            live = [i for i, s in enumerate(slots) if s is not None]
            # The next round is enqueued before the pending round's report is
            # read when no request waits for a slot and the pending round cannot
            # end every sequence (one that ignores EOS has more than K + 1
            # tokens left), so the host's bookkeeping overlaps the device.  A
            # sequence that ends in the pending round is inactive on the device
            # by then, and the round launched over it skips it.
            launch = bool(live) and (pending is None or (
                not self.scheduler.waiting and any(slots[i].ignore_eos and left[i] > K + 1 for i in live)))
            cur = None
            if launch:
                B = r.bucket_for(max(live) + 1)
                r.launch(B, rep_slot)
                cur = (B, rep_slot)
                rep_slot ^= 1
                rounds += 1
            if pending is not None:
                act, com, dr, mdl = r.collect(*pending).tolist()
                self.spec_stats["rounds"] += 1
                fallback = 0
                for i in range(pending[0]):
                    if slots[i] is None:
                        continue
                    if self.spec_method != "none" and dr[i] > 0:
                        self.spec_stats["drafted_tokens"] += dr[i]
                        self.spec_stats["accepted_tokens"] += com[i]
                        fallback += mdl[i]
                    decode_tokens += com[i]
                    left[i] -= com[i]
                if self.spec_method == "hybrid" and fallback:
                    self.spec_stats["model_fallback_rounds"] += 1
                    self.spec_stats["model_fallback_seqs"] += fallback
                # a slot that ended is inactive in any round in flight; reading
                # its history waits for that round on the stream
                for i in range(pending[0]):
                    if slots[i] is not None and not act[i]:
                        finish(i)
            pending = cur
        torch.cuda.synchronize(self.device)
        t_end = time.perf_counter()
        token_ids = [s.completion_token_ids for s in requests]
        output_tokens = sum(len(t) for t in token_ids)
        total = t_end - t0
        decode_s = max(total - prefill_s, 1e-9)
        metrics = {
            "total_s": total,
            "ttft_s": (first_token_t or t_end) - t0,
            "prefill_tokens": prefill_tokens,
            "decode_tokens": decode_tokens,
            "output_tokens": output_tokens,
            "prefix_cache": self.block_manager.cache_stats(),
            "spec_decoding": dict(self.spec_stats),
            # this build's additions
            "prefill_s": prefill_s,
            "decode_s": decode_s,
            "rounds": rounds,
            "decode_tok_per_s": decode_tokens / decode_s,
            "output_tok_per_s": output_tokens / max(total, 1e-9),
        }
        return {"token_ids": token_ids, "outputs": [{"token_ids": t} for t in token_ids], "metrics": metrics}
