"""Speculative-decoding engine over the device-resident verification round.

Keeps the reference's SpecLLMEngine configuration keys and spec metrics
(src/myvllm/spec_engine/spec_llm_engine.py:32-102, :305-312):
``spec_method`` ("ngram", or "none" for plain decoding through the same
round with drafting off), ``num_speculative_tokens``, ``ngram_min_size``,
``ngram_max_size``, ``max_num_sequences``, ``max_model_length``,
``block_size``, ``world_size`` (must be 1, :34-35), ``enforce_eager`` /
``capture_verify``; ``metrics["spec_decoding"]`` holds ``rounds``,
``drafted_tokens``, ``accepted_tokens`` and ``fallback_rounds``, cumulative
over calls as in the reference.  The model is a random-init Qwen3 of the
shape in ``config["model_config"]`` (no checkpoint loading: :104-137 and
utils/loader.py fetch weights by name, which this build does not do).

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

PREFILL_ROWS = 64  # GQA group x query rows one verify-attention call handles


class SpecLLMEngine:
    def __init__(self, config: dict):
        assert config.get("world_size", 1) == 1, "speculative decoding currently supports world_size == 1"
        self.spec_method = config.get("spec_method", "ngram")
        if self.spec_method not in ("ngram", "none"):
            raise ValueError(f"spec_method {self.spec_method!r}: this build runs 'ngram' and 'none'")
        self.num_speculative_tokens = config.get("num_speculative_tokens", 5)
        self.min_ngram = config.get("ngram_min_size", 2)
        self.max_ngram = config.get("ngram_max_size", 8)
        self.max_num_sequences = config.get("max_num_sequences", 8)
        self.max_model_length = config.get("max_model_length", 4096)
        self.block_size = config.get("block_size", 256)
        self.eos = config.get("eos_token_id", -1)
        self.device = torch.device(config.get("device", "cuda"))
        cfg = config.get("model_config") or Qwen3Config()
        self.model = Qwen3Verify(cfg, self.device, seed=config.get("seed", 0))
        K = self.num_speculative_tokens
        self.history_len = self.max_model_length + K + 1
        self.max_blocks = math.ceil(self.history_len / self.block_size)
        num_blocks = config.get("num_kvcache_blocks", self.max_num_sequences * self.max_blocks)
        self.block_manager = BlockManager(num_blocks, self.block_size)
        self.model.allocate_kv_cache(num_blocks, self.block_size)
        self.round = VerifyRound(self.model, self.max_num_sequences, K, self.min_ngram, self.max_ngram,
                                 self.history_len, self.max_blocks, self.eos, draft=self.spec_method != "none")
        eager = config.get("enforce_eager", False) or not config.get("capture_verify", True)
        if not eager:
            self.round.capture()
        self.spec_stats = {"method": self.spec_method, "num_speculative_tokens": K, "rounds": 0,
                           "drafted_tokens": 0, "accepted_tokens": 0, "fallback_rounds": 0}

    # ------------------------------------------------------------------ prefill
    @torch.inference_mode()
    def _prefill(self, seq: Sequence) -> int:
        """KV of the prompt (chunks of prompt rows through the verify forward)
        and the first completion token (greedy: argmax of the last prompt
        row), as the reference's prefill + sampler produce it."""
        dev = self.device
        table = torch.tensor(seq.block_table, dtype=torch.int32, device=dev).unsqueeze(0)
        bs = self.block_size
        logits = None
        n = len(seq.token_ids)
        cfg = self.model.cfg
        chunk = PREFILL_ROWS // (cfg.num_heads // cfg.num_kv_heads)
        for p0 in range(0, n, chunk):
            p1 = min(n, p0 + chunk)
            pos = torch.arange(p0, p1, dtype=torch.int64, device=dev)
            ids = torch.tensor(seq.token_ids[p0:p1], dtype=torch.int64, device=dev)
            pages = table[0, (pos // bs)].to(torch.int64)
            slots = pages * bs + pos % bs
            ctx = torch.tensor([p1], dtype=torch.int64, device=dev)
            cu = torch.tensor([0, p1 - p0], dtype=torch.int32, device=dev)
            logits = self.model.forward(ids, pos, slots, table, ctx, cu, p1 - p0)
        return int(logits[-1].argmax())

    # ---------------------------------------------------------------- generate
    @torch.inference_mode()
    def generate(self, prompts: list[list[int]], sampling_params: SamplingParams | list[SamplingParams]) -> dict:
        if len(prompts) > self.max_num_sequences:
            raise ValueError(f"{len(prompts)} prompts exceed max_num_sequences={self.max_num_sequences}")
        params = sampling_params if isinstance(sampling_params, list) else [sampling_params] * len(prompts)
        for sp in params:
            if sp.temperature > 1e-6:
                raise ValueError("this build's device round accepts greedily (temperature 0)")
        K = self.num_speculative_tokens
        r = self.round
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
        rounds = 0
        decode_tokens = 0
        while live:
            B = r.bucket_for(max(live) + 1)
            rep = r.run(B)
            rounds += 1
            act, com, dr = rep[0].tolist(), rep[1].tolist(), rep[2].tolist()
            self.spec_stats["rounds"] += 1
            for i in live:
                if self.spec_method != "none" and dr[i] > 0:
                    self.spec_stats["drafted_tokens"] += dr[i]
                    self.spec_stats["accepted_tokens"] += com[i]
                decode_tokens += com[i]
            live = [i for i in live if act[i]]
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
