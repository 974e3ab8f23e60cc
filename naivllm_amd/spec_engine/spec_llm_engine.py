"""Speculative-decoding engine over the device-resident verification round.

Keeps the reference's SpecLLMEngine configuration keys and spec metrics
(src/myvllm/spec_engine/spec_llm_engine.py:32-102, :305-312):
``spec_method`` ("ngram", "model", "hybrid", or "none" for plain decoding
through the same round with drafting off), ``num_speculative_tokens``,
``ngram_min_size``, ``ngram_max_size``, ``max_num_sequences``,
``max_model_length``, ``block_size``, ``world_size`` (must be 1, :34-35),
``enforce_eager`` / ``capture_verify``; ``metrics["spec_decoding"]`` holds
``rounds``, ``drafted_tokens``, ``accepted_tokens`` and ``fallback_rounds``
(cumulative over calls as in the reference), plus
``model_fallback_rounds`` / ``model_fallback_seqs`` for a hybrid drafter
(:305-312).  The target is a random-init Qwen3 of the shape in
``config["model_config"]``; the model / hybrid drafter a random-init Qwen3
of ``config["draft_model_config"]`` (Qwen3-0.6B by default) that shares the
target's vocabulary, pages and block tables (no checkpoint loading: :104-137
and utils/loader.py fetch weights by name, which this build does not do).

Sampling: a request with temperature <= 1e-6 is decoded greedily; any
other temperature samples the first token, the model drafts and the
acceptance (min(1, p_t/p_d) with residual resampling) from torch's device
generator, seeded from ``config["seed"]``.  Rounds of greedy-only batches
run the greedy graphs; a batch with a sampled request runs the stochastic
graphs (built on first use).

Scheduling is a fixed batch: ``generate`` admits up to max_num_sequences
prompts, prefills them, and runs rounds until every sequence finished;
finished sequences stay in their slot as inactive rows, and the batch moves
to a smaller captured bucket when the active ones fit one.
"""

from __future__ import annotations

import math
import time

import torch

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.sequence import Sequence, SequenceStatus
from naivllm_amd.engine.verify_round import VerifyRound
from naivllm_amd.layers.qwen3 import Qwen3Config, Qwen3Verify
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine.rejection_sampler import GREEDY_TEMPERATURE, sample

PREFILL_ROWS = 64  # GQA group x query rows one verify-attention call handles


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
        self.max_model_length = config.get("max_model_length", 4096)
        self.block_size = config.get("block_size", 256)
        self.eos = config.get("eos_token_id", -1)
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
        K = self.num_speculative_tokens
        self.history_len = self.max_model_length + K + 1
        self.max_blocks = math.ceil(self.history_len / self.block_size)
        num_blocks = config.get("num_kvcache_blocks", self.max_num_sequences * self.max_blocks)
        self.block_manager = BlockManager(num_blocks, self.block_size)
        self.model.allocate_kv_cache(num_blocks, self.block_size)
        if self.draft_model is not None:
            self.draft_model.allocate_kv_cache(num_blocks, self.block_size)
        self.eager = config.get("enforce_eager", False) or not config.get("capture_verify", True)
        self.rounds: dict[bool, VerifyRound] = {}  # greedy / stochastic round, built on first use
        self.spec_stats = {"method": self.spec_method, "num_speculative_tokens": K, "rounds": 0,
                           "drafted_tokens": 0, "accepted_tokens": 0, "fallback_rounds": 0}
        if self.spec_method == "hybrid":
            self.spec_stats.update(model_fallback_rounds=0, model_fallback_seqs=0)

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

    # ------------------------------------------------------------------ prefill
    @torch.inference_mode()
    def _prefill(self, seq: Sequence) -> int:
        """KV of the prompt (chunks of prompt rows through the verify
        forward; mirrored into the draft model's cache when there is one,
        spec_llm_engine.py:147-151) and the first completion token, sampled
        from the last prompt row as the reference's prefill + sampler
        (layers/sampler.py:14-24) do."""
        dev = self.device
        table = torch.tensor(seq.block_table, dtype=torch.int32, device=dev).unsqueeze(0)
        bs = self.block_size
        logits = None
        n = len(seq.token_ids)
        cfg = self.model.cfg
        chunk = PREFILL_ROWS // (cfg.num_heads // cfg.num_kv_heads)
        if self.draft_model is not None:
            dc = self.draft_model.cfg
            chunk = min(chunk, PREFILL_ROWS // (dc.num_heads // dc.num_kv_heads))
        for p0 in range(0, n, chunk):
            p1 = min(n, p0 + chunk)
            pos = torch.arange(p0, p1, dtype=torch.int64, device=dev)
            ids = torch.tensor(seq.token_ids[p0:p1], dtype=torch.int64, device=dev)
            pages = table[0, (pos // bs)].to(torch.int64)
            slots = pages * bs + pos % bs
            ctx = torch.tensor([p1], dtype=torch.int64, device=dev)
            cu = torch.tensor([0, p1 - p0], dtype=torch.int32, device=dev)
            logits = self.model.forward(ids, pos, slots, table, ctx, cu, p1 - p0)
            if self.draft_model is not None:
                self.draft_model.forward(ids, pos, slots, table, ctx, cu, p1 - p0)
        last = logits[-1:]
        if seq.temperature <= GREEDY_TEMPERATURE:
            return int(last.argmax())
        noise = torch.empty(1, last.shape[-1], dtype=torch.float32, device=dev).exponential_(1).clamp_min_(1e-10)
        temp = torch.full((1,), float(seq.temperature), dtype=torch.float32, device=dev)
        return int(sample(last, temp, noise)[0])

    # ---------------------------------------------------------------- generate
    @torch.inference_mode()
    def generate(self, prompts: list[list[int]], sampling_params: SamplingParams | list[SamplingParams]) -> dict:
        if len(prompts) > self.max_num_sequences:
            raise ValueError(f"{len(prompts)} prompts exceed max_num_sequences={self.max_num_sequences}")
        params = sampling_params if isinstance(sampling_params, list) else [sampling_params] * len(prompts)
        K = self.num_speculative_tokens
        r = self._round(any(sp.temperature > GREEDY_TEMPERATURE for sp in params))
        t0 = time.perf_counter()
        seqs = []
        for slot, (prompt, sp) in enumerate(zip(prompts, params)):
            seq = Sequence(prompt, sp)
            cap = min(len(prompt) + sp.max_tokens, sp.max_model_length or self.max_model_length,
                      self.max_model_length)
            if len(prompt) >= self.history_len - K - 1:
                raise ValueError("prompt longer than max_model_length")
            self.block_manager.allocate(seq)
            self.block_manager.ensure_capacity(seq, cap + K + 1)
            seq.status = SequenceStatus.RUNNING
            first = self._prefill(seq)
            seq.append_token(first)
            r.history[slot, :seq.num_tokens] = torch.tensor(seq.token_ids, dtype=torch.int32, device=self.device)
            r.hist_len[slot] = seq.num_tokens
            r.prompt_len[slot] = seq.num_prompt_tokens
            r.max_tokens[slot] = sp.max_tokens
            r.max_len[slot] = sp.max_model_length or self.max_model_length
            r.ignore_eos[slot] = int(sp.ignore_eos)
            r.temperature[slot] = float(sp.temperature)
            r.block_tables[slot].fill_(-1)
            r.block_tables[slot, :len(seq.block_table)] = torch.tensor(seq.block_table, dtype=torch.int32,
                                                                       device=self.device)
            done = (seq.num_completion_tokens >= sp.max_tokens or (not sp.ignore_eos and first == self.eos))
            r.active[slot] = 0 if done else 1
            seqs.append(seq)
        for slot in range(len(seqs), r.max_batch):
            r.active[slot] = 0
            r.hist_len[slot] = 0
        torch.cuda.synchronize(self.device)
        t_prefill = time.perf_counter()

        live = [i for i, s in enumerate(seqs) if int(r.active[i])]
        # tokens each sequence may still commit (max_tokens and length caps);
        # a round commits at most K + 1
        left = {i: min(params[i].max_tokens - seqs[i].num_completion_tokens,
                       (params[i].max_model_length or self.max_model_length) - seqs[i].num_tokens) for i in live}
        rounds = 0
        decode_tokens = 0
        pending = None  # (bucket, report slot) of a launched round whose report is unread
        slot = 0
        while live or pending is not None:
            # The next round is enqueued before the pending round's report is
            # read when the pending round cannot end every sequence (one that
            # ignores EOS has more than K + 1 tokens left), so the host's
            # bookkeeping overlaps the device.  A sequence that ends in the
            # pending round is inactive on the device by then, and the round
            # launched over it skips it (the bucket may be one size too large
            # for that round).
            launch = bool(live) and (pending is None or any(params[i].ignore_eos and left[i] > K + 1 for i in live))
            if launch:
                B = r.bucket_for(max(live) + 1)
                r.launch(B, slot)
                cur = (B, slot)
                slot ^= 1
                rounds += 1
            if pending is not None:
                rep = r.collect(*pending)
                act, com, dr, mdl = rep.tolist()
                self.spec_stats["rounds"] += 1
                fallback = 0
                for i in live:
                    if self.spec_method != "none" and dr[i] > 0:
                        self.spec_stats["drafted_tokens"] += dr[i]
                        self.spec_stats["accepted_tokens"] += com[i]
                        fallback += mdl[i]
                    decode_tokens += com[i]
                    left[i] -= com[i]
                if self.spec_method == "hybrid" and fallback:
                    self.spec_stats["model_fallback_rounds"] += 1
                    self.spec_stats["model_fallback_seqs"] += fallback
                live = [i for i in live if act[i]]
            pending = cur if launch else None
        torch.cuda.synchronize(self.device)
        t_end = time.perf_counter()

        hist = r.history[:len(seqs)].cpu()
        lens = r.hist_len[:len(seqs)].cpu().tolist()
        outputs = []
        for i, seq in enumerate(seqs):
            seq.token_ids = hist[i, :lens[i]].tolist()
            seq.num_tokens = lens[i]
            seq.last_token = seq.token_ids[-1]
            seq.status = SequenceStatus.FINISHED
            self.block_manager.deallocate(seq)
            outputs.append({"token_ids": seq.completion_token_ids})
        gen = sum(len(o["token_ids"]) for o in outputs)
        metrics = {
            "total_s": t_end - t0,
            "prefill_s": t_prefill - t0,
            "decode_s": t_end - t_prefill,
            "output_tokens": gen,
            "decode_tokens": decode_tokens,
            "rounds": rounds,
            "decode_tok_per_s": decode_tokens / max(t_end - t_prefill, 1e-9),
            "spec_decoding": dict(self.spec_stats),
        }
        return {"outputs": outputs, "metrics": metrics}
