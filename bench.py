"""Benchmark of the verify round's dominant kernel on one MI355X.

One step = the verify-attention work of one verification round of
Qwen3-0.6B: 28 layers, each a paged verify-attention
call over that layer's own KV cache (B=8, 16Q/8KV heads, d=128, bf16,
256-token pages, contexts uniform in [1200, 1300], K=8 drafts so 9 query
rows per sequence).  The 28 distinct caches (~1.9 GB) rotate the working set
far past the 256 MB Infinity Cache, so the bandwidth is HBM bandwidth.

Prints one JSON line (rank 0).  ``value`` = algorithmic bytes per
verify-attention call / average call duration, the duration from HIP
events on the stream the kernels run on, over the timed steps.  Each step
is one replay of a hipGraph holding the 28 calls, as in the graphed verify
round.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from naivllm_amd.layers.attention import paged_attention_verify  # noqa: E402
from naivllm_amd.utils import synth  # noqa: E402

METRIC = "verify-attn HBM GB/s (% of peak) + accepted tok/s, Qwen3-0.6B K=8 b1/b8"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def algorithmic_bytes(ctx_lens, T, H, Hkv, D, elt, max_blocks) -> int:
    """KV read once + Q read + O written + metadata (block table, context
    lengths, cu_seqlens, positions)."""
    B = len(ctx_lens)
    kv = sum(ctx_lens) * Hkv * D * 2 * elt
    return kv + 2 * T * H * D * elt + 4 * B * max_blocks + 8 * B + 4 * (B + 1) + 8 * T


def algorithmic_flops(ctx_lens, q_rows_per_seq, H, D) -> int:
    return 4 * q_rows_per_seq * D * H * sum(ctx_lens)


class Workload:
    def __init__(self, config: int, layers: int, seed: int, device, batch: int = 8):
        self.config = config
        if config == 2:
            self.B, self.H, self.Hkv, self.D, self.bs, self.K = batch, 16, 8, 128, 256, 8
            self.ctx = synth.config2_ctx_lens(seed, self.B)
            self.layers = layers
            pool_pages = max(64, sum((c + self.bs - 1) // self.bs for c in self.ctx))
            name = f"verify-attention, Qwen3-0.6B layer shape, b{batch} bf16, L~U[1200,1300], K=8, 28 layers"
        elif config == 4:
            self.B, self.H, self.Hkv, self.D, self.bs, self.K = 16, 32, 8, 128, 256, 8
            self.ctx = [int(x) for x in synth.randint(seed, 7, 16, 16384, 32769)]
            self.layers = max(2, min(layers, 2))
            pool_pages = 1700
            name = "verify-attention, Qwen3-8B layer shape, b16 bf16, L~U[16k,32k], K=8, 2 rotating pools"
        else:
            raise SystemExit(f"config {config} is not a bench workload (2 or 4)")
        self.name = name
        self.rows = self.K + 1
        self.T = self.B * self.rows
        pages = [(c + self.bs - 1) // self.bs for c in self.ctx]
        self.max_blocks = max(pages)
        perm = synth.randperm(seed, 1, pool_pages)
        bt = np.full((self.B, self.max_blocks), -1, dtype=np.int32)
        off = 0
        for b in range(self.B):
            bt[b, :pages[b]] = perm[off:off + pages[b]]
            off += pages[b]
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        shape = (pool_pages, self.bs, self.Hkv, self.D)
        self.k_caches = [torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16) for _ in range(self.layers)]
        self.v_caches = [torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16) for _ in range(self.layers)]
        self.q = torch.randn(self.T, self.H, self.D, generator=g, device=device, dtype=torch.bfloat16)
        self.out = torch.empty_like(self.q)
        self.block_tables = torch.from_numpy(bt).to(device)
        self.context_lens = torch.tensor(self.ctx, dtype=torch.int64, device=device)
        self.cu = torch.arange(0, self.T + 1, self.rows, dtype=torch.int32, device=device)
        pos = np.concatenate([np.arange(c - self.rows, c) for c in self.ctx])
        self.positions = torch.from_numpy(pos).to(device)
        self.scale = 1.0 / np.sqrt(self.D)
        self.bytes = algorithmic_bytes(self.ctx, self.T, self.H, self.Hkv, self.D, 2, self.max_blocks)
        self.flops = algorithmic_flops(self.ctx, self.rows, self.H, self.D)

    def call(self, layer: int, split: int):
        paged_attention_verify(self.q, self.k_caches[layer], self.v_caches[layer], self.block_tables,
                               self.context_lens, self.cu, self.positions, self.scale, self.H, self.Hkv, self.D,
                               self.bs, 16, max_q_len=self.rows, kv_split_tokens=split, out=self.out)

    def step(self, split: int):
        for layer in range(self.layers):
            self.call(layer, split)


def traffic_profile(workload_config: int) -> str:
    return os.path.join(ROOT, "profiles", f"verify_attn_config{workload_config}_traffic.md")


def measured_traffic(workload_config: int):
    """HBM bytes per verify-attention launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (copy-calibrated) of that workload, or
    None when no such profile is committed."""
    path = traffic_profile(workload_config)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes:"):
            return int(line.split(":")[1])
    return None


def e2e_round(batches=(1, 2, 4, 8), tokens: int = 48, K: int = 8) -> dict:
    """the whole greedy n-gram verification round of a
    random-init Qwen3-0.6B (28 layers, bf16) at batch 1/2/4/8, one hipGraph
    replay per round per batch bucket.  Reported per batch: decode tokens
    per second over the rounds (prefill excluded), output tokens per second
    over the whole request (prefill included, as the reference's output_tps),
    time to first token, and the prompt tokens prefilled (the batch's
    requests share their 1200-token document, whose full pages the prefix
    cache serves after the first request).  Each batch runs on a fresh
    engine, so no earlier batch warms its cache."""
    from naivllm_amd.sampling_parameters import SamplingParams
    from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine

    sp = SamplingParams(temperature=0.0, max_tokens=tokens, ignore_eos=True)
    out = {}
    for b in batches:
        eng = SpecLLMEngine(dict(spec_method="ngram", num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4,
                                 max_num_sequences=max(batches), max_model_length=1200 + 16 + tokens + 64,
                                 block_size=256, seed=0))
        eng.generate(synth.config3_prompts(1, seed=99), SamplingParams(temperature=0.0, max_tokens=4,
                                                                        ignore_eos=True))  # graphs captured, warm
        before = dict(eng.spec_stats)
        res = eng.generate(synth.config3_prompts(b), sp)
        m = res["metrics"]
        st = m["spec_decoding"]
        drafted = st["drafted_tokens"] - before["drafted_tokens"]
        accepted = st["accepted_tokens"] - before["accepted_tokens"]
        out[f"b{b}"] = {
            "decode_tok_s": round(m["decode_tok_per_s"], 1),
            "output_tok_s": round(m["output_tok_per_s"], 1),
            "ttft_s": round(m["ttft_s"], 4),
            "decode_ms_per_round": round(1e3 * m["decode_s"] / max(m["rounds"], 1), 3),
            "rounds": m["rounds"],
            "tokens_per_round": round(m["decode_tokens"] / max(m["rounds"], 1), 3),
            "drafted": drafted,
            "accepted": accepted,
            "prefill_tokens": m["prefill_tokens"],
            "prefill_s": round(m["prefill_s"], 4),
            "output_tokens": m["output_tokens"],
        }
        print(f"[bench] e2e b{b}: {out[f'b{b}']}", file=sys.stderr, flush=True)
        eng.exit()
        del eng
        torch.cuda.empty_cache()
    return out


def e2e_self_draft(batches=(1, 8), tokens: int = 55, K: int = 8) -> dict:
    """The K=8 regime with every draft accepted.  Random-init Qwen3-0.6B
    decodes greedily into one repeated token, and for a constant run the
    n-gram lookup (the reference's rfind from the most recent match) can
    only ever continue with one token, so n-gram rounds carry at most one
    draft.  Here the model drafter runs the target's own weights (same
    seed): its greedy drafts are the target's greedy tokens, so each round
    verifies and commits K drafts plus the bonus token through the same
    captured round (K GPU-resident draft steps, one 9-row verify forward,
    greedy acceptance, commit).  Config-3 prompts, b1 and b8, each batch on
    a fresh engine after a warm-up request; 55 output tokens (the prefill's
    first token and 6 whole rounds of K + 1), so no round is cut short by
    max_tokens.  Acceptance = accepted drafts / drafted, an accepted draft
    being a committed token other than each sequence's per-round bonus or
    correction token."""
    from naivllm_amd.layers.qwen3 import Qwen3Config
    from naivllm_amd.sampling_parameters import SamplingParams
    from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine

    sp = SamplingParams(temperature=0.0, max_tokens=tokens, ignore_eos=True)
    out = {"drafter": "model drafter with the target's own weights (Qwen3-0.6B, same seed): self-speculation"}
    for b in batches:
        eng = SpecLLMEngine(dict(spec_method="model", num_speculative_tokens=K, model_config=Qwen3Config.qwen3_0_6b(),
                                 draft_model_config=Qwen3Config.qwen3_0_6b(), draft_seed=0, seed=0,
                                 max_num_sequences=max(batches), max_model_length=1200 + 16 + tokens + 64,
                                 block_size=256))
        eng.generate(synth.config3_prompts(1, seed=99), SamplingParams(temperature=0.0, max_tokens=4,
                                                                        ignore_eos=True))  # graphs captured, warm
        before = dict(eng.spec_stats)
        res = eng.generate(synth.config3_prompts(b), sp)
        m = res["metrics"]
        st = m["spec_decoding"]
        drafted = st["drafted_tokens"] - before["drafted_tokens"]
        accepted = st["accepted_tokens"] - before["accepted_tokens"]
        rounds = max(m["rounds"], 1)
        out[f"b{b}"] = {
            "decode_tok_s": round(m["decode_tok_per_s"], 1),
            "output_tok_s": round(m["output_tok_per_s"], 1),
            "decode_ms_per_round": round(1e3 * m["decode_s"] / rounds, 3),
            "rounds": m["rounds"],
            "tokens_per_round": round(m["decode_tokens"] / rounds, 3),
            "drafted": drafted,
            "committed": accepted,
            "acceptance": round((accepted - m["rounds"] * b) / max(drafted, 1), 4) if drafted else None,
            "output_tokens": m["output_tokens"],
        }
        print(f"[bench] self-draft b{b}: {out[f'b{b}']}", file=sys.stderr, flush=True)
        eng.exit()
        del eng
        torch.cuda.empty_cache()
    return out


def e2e_cascade(batches=(1, 8), tokens: int = 48, K: int = 8) -> dict:
    """a random-init Qwen3-0.6B drafter feeding a
    random-init Qwen3-8B target (36 layers, hidden 4096, 32Q/8KV, bf16)
    through the hybrid drafter (n-gram first, K = 8 GPU-resident draft
    steps otherwise), one 9-row verify forward and min(1, p_t/p_d)
    acceptance at temperature 1.0; 1200-token prefix, 48 output tokens.
    Decode tokens per second over the rounds (one hipGraph replay per
    round), output tokens per second over the whole request and time to
    first token, each batch on a fresh engine."""
    from naivllm_amd.layers.qwen3 import Qwen3Config
    from naivllm_amd.sampling_parameters import SamplingParams
    from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine

    sp = SamplingParams(temperature=1.0, max_tokens=tokens, ignore_eos=True)
    out = {}
    for b in batches:
        eng = SpecLLMEngine(dict(spec_method="hybrid", num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4,
                                 model_config=Qwen3Config.qwen3_8b(), draft_model_config=Qwen3Config.qwen3_0_6b(),
                                 max_num_sequences=max(batches), max_model_length=1200 + 16 + tokens + 64,
                                 block_size=256, seed=5))
        eng.generate(synth.config3_prompts(1, seed=99), SamplingParams(temperature=1.0, max_tokens=4,
                                                                        ignore_eos=True))  # graphs captured, warm
        before = dict(eng.spec_stats)
        res = eng.generate(synth.config3_prompts(b, seed=5), sp)
        m = res["metrics"]
        st = m["spec_decoding"]
        out[f"b{b}"] = {
            "decode_tok_s": round(m["decode_tok_per_s"], 1),
            "output_tok_s": round(m["output_tok_per_s"], 1),
            "ttft_s": round(m["ttft_s"], 4),
            "decode_ms_per_round": round(1e3 * m["decode_s"] / max(m["rounds"], 1), 3),
            "rounds": m["rounds"],
            "tokens_per_round": round(m["decode_tokens"] / max(m["rounds"], 1), 3),
            "drafted": st["drafted_tokens"] - before["drafted_tokens"],
            "accepted": st["accepted_tokens"] - before["accepted_tokens"],
            "model_fallback_seqs": st["model_fallback_seqs"] - before["model_fallback_seqs"],
            "prefill_tokens": m["prefill_tokens"],
            "prefill_s": round(m["prefill_s"], 4),
            "output_tokens": m["output_tokens"],
        }
        print(f"[bench] cascade b{b}: {out[f'b{b}']}", file=sys.stderr, flush=True)
        eng.exit()
        del eng
        torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown CPU"


def _median_seconds(fn, warmup: int = 5, reps: int = 20) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_baseline() -> dict:
    """BASELINE config 1 on the host's cores (the torch-CPU restatement of
    the reference's path, oracle/torch_cpu.py): one verify-attention call
    (b1 fp32, 16Q/8KV, d 128, L = 1248 in 5 pages of a seeded-permuted
    64-page pool, 9 query rows; layers/attention.py:328-363) plus the greedy
    acceptance of 8 drafts over [9, 151936] fp32 logits ~ N(0, 2^2) whose
    first 5 drafts are the argmax (spec_llm_engine.py:224-227,
    rejection_sampler.py:25-36).  5 warm-up reps, then the median of 20,
    with every host thread and with one.  Also the config-2 attention call
    (b8 bf16), the GPU metric's workload, with every thread."""
    from oracle import torch_cpu

    H, Hkv, D, bs, R, V = 16, 8, 128, 256, 9, 151936
    g = torch.Generator().manual_seed(1)
    kc = torch.randn(64, bs, Hkv, D, generator=g)
    vc = torch.randn(64, bs, Hkv, D, generator=g)
    q = torch.randn(R, H, D, generator=g)
    bt = torch.randperm(64, generator=g)[:5].to(torch.int32)[None]
    L = 1248
    args1 = (q, kc, vc, bt, torch.tensor([L]), torch.tensor([0, R], dtype=torch.int32), torch.arange(L - R, L),
             1 / np.sqrt(D), H, Hkv)
    logits = torch.randn(R, V, generator=g) * 2.0
    am = logits.argmax(-1).tolist()
    drafts = [am[:5] + [int(x) for x in torch.randint(0, V, (3,), generator=g)]]
    accepted = torch_cpu.greedy_accept(drafts, logits, R)
    attn_bytes = L * Hkv * D * 2 * 4 + 2 * R * H * D * 4 + 4 * 5 + 8 + 8 + 8 * R
    accept_bytes = R * V * 4
    step = lambda: (torch_cpu.paged_verify_attention(*args1), torch_cpu.greedy_accept(drafts, logits, R))  # noqa: E731
    threads = os.cpu_count() or 1
    out = {"unit": "GB/s", "kind": "port", "cpu": cpu_model()}
    for n in (threads, 1):
        torch.set_num_threads(n)
        sec = _median_seconds(step)
        key = "all_threads" if n == threads else "one_thread"
        out[key] = {"threads": n, "median_ms": round(sec * 1e3, 3),
                    "GBs": round((attn_bytes + accept_bytes) / sec / 1e9, 3)}
    torch.set_num_threads(threads)
    out["value"] = out["all_threads"]["GBs"]
    out["cores"] = threads
    out["sample"] = (f"BASELINE config 1: one verify-attention call (b1 fp32, L=1248, 16Q/8KV, d128) + greedy "
                     f"acceptance over [9, 151936] fp32 logits ({len(accepted[0])} tokens accepted), median of 20 "
                     f"after 5 warm-ups on {out['cpu']}; {attn_bytes + accept_bytes} algorithmic bytes per step")
    # config 2's attention call (the GPU metric's workload), every thread
    ctx2 = synth.config2_ctx_lens(2, 8)
    pages = [(c + bs - 1) // bs for c in ctx2]
    g2 = torch.Generator().manual_seed(2)
    nb = sum(pages) + 4
    kc2 = torch.randn(nb, bs, Hkv, D, generator=g2).to(torch.bfloat16)
    vc2 = torch.randn(nb, bs, Hkv, D, generator=g2).to(torch.bfloat16)
    q2 = torch.randn(8 * R, H, D, generator=g2).to(torch.bfloat16)
    bt2 = torch.full((8, max(pages)), -1, dtype=torch.int32)
    off = 0
    for b in range(8):
        bt2[b, :pages[b]] = torch.arange(off, off + pages[b], dtype=torch.int32)
        off += pages[b]
    args2 = (q2, kc2, vc2, bt2, torch.tensor(ctx2), torch.arange(0, 8 * R + 1, R, dtype=torch.int32),
             torch.cat([torch.arange(c - R, c) for c in ctx2]), 1 / np.sqrt(D), H, Hkv)
    sec = _median_seconds(lambda: torch_cpu.paged_verify_attention(*args2))
    nbytes = algorithmic_bytes(ctx2, 8 * R, H, Hkv, D, 2, max(pages))
    out["config2_attention"] = {"threads": threads, "median_ms": round(sec * 1e3, 3),
                                "GBs": round(nbytes / sec / 1e9, 3)}
    return out


def _graph_us(step, calls_per_step: int, steps: int = 50, warmup: int = 5) -> float:
    """Average duration of one call: ``step`` (calls_per_step launches on
    the current stream) is captured as a hipGraph and replayed; HIP events
    on that stream bracket the timed replays."""
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * calls_per_step)


def ceilings(wl: "Workload") -> dict:
    """Load-only ceilings of the metric's workload, timed like the metric:
    the verify-attention K/V bytes read in the key-split kernel's access
    pattern with nothing computed (nsv_verify_attention_load_floor, same
    28 rotating pools, the plan's splits), and a contiguous read of the
    same byte count from 28 rotating flat buffers (nsv_stream_read, 1024
    workgroups)."""
    from naivllm_amd import _lib
    from naivllm_amd.layers.attention import verify_attention_plan

    h = _lib.lib()
    dev = wl.q.device
    kind, splits = verify_attention_plan(wl.B, wl.H, wl.Hkv, wl.D, wl.bs, wl.max_blocks, wl.rows, torch.bfloat16)
    splits = splits if kind == "key-split" else 4
    sink = torch.zeros(65536, dtype=torch.int32, device=dev)
    kv_bytes = sum(wl.ctx) * wl.Hkv * wl.D * 2 * 2

    def floor_step():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(wl.layers):
            rc = h.nsv_verify_attention_load_floor(wl.k_caches[layer].data_ptr(), wl.v_caches[layer].data_ptr(),
                                                  wl.block_tables.data_ptr(), wl.context_lens.data_ptr(), wl.B,
                                                  wl.Hkv, wl.D, wl.bs, wl.max_blocks, splits, sink.data_ptr(), s)
            _lib.check(rc, "load floor")
    floor_us = _graph_us(floor_step, wl.layers)
    flat = [torch.ones(kv_bytes, dtype=torch.uint8, device=dev) for _ in range(wl.layers)]

    def stream_step():
        s = torch.cuda.current_stream().cuda_stream
        for layer in range(wl.layers):
            _lib.check(h.nsv_stream_read(flat[layer].data_ptr(), kv_bytes, 1024, sink.data_ptr(), s), "stream")
    stream_us = _graph_us(stream_step, wl.layers)
    del flat
    torch.cuda.empty_cache()
    return {"kv_bytes": kv_bytes, "splits": splits,
            "load_floor_us": round(floor_us, 3), "load_floor_GBs": round(kv_bytes / floor_us / 1e3, 1),
            "stream_us": round(stream_us, 3), "stream_GBs": round(kv_bytes / stream_us / 1e3, 1)}


def cu_intake(per_mib=(1,), groups=(32, 64, 128, 256)) -> dict:
    """How fast a few CUs take in bytes, against the whole chip: G
    workgroups of 512 threads each read their own contiguous per-MiB slice
    (nsv_stream_read, 16-byte non-temporal loads), graph-replayed over 8
    rotating slices of a 2 GiB buffer so that every call reads from HBM.
    Reported per G: us per call, total GB/s and GB/s per workgroup (one
    workgroup per CU at these counts); and the time per call of a graph of
    64 one-workgroup, one-load kernels (the floor of a dependent launch)."""
    from naivllm_amd import _lib

    h = _lib.lib()
    dev = torch.device("cuda:0")
    buf = torch.ones(2 << 30, dtype=torch.uint8, device=dev)
    sink = torch.zeros(65536, dtype=torch.int32, device=dev)
    out = {}
    for mib in per_mib:
        for g in groups:
            nbytes = g * (mib << 20)
            slots = min(8, (2 << 30) // nbytes)

            def step():
                s = torch.cuda.current_stream().cuda_stream
                for i in range(8):
                    off = (i % slots) * nbytes
                    _lib.check(h.nsv_stream_read(buf.data_ptr() + off, nbytes, g, sink.data_ptr(), s), "stream")
            us = _graph_us(step, 8, steps=20)
            out[f"{g}x{mib}MiB"] = {"us": round(us, 2), "GBs": round(nbytes / us / 1e3, 1),
                                    "GBs_per_workgroup": round(nbytes / g / us / 1e3, 1)}

    # the floor of one dependent launch in a graph: one workgroup, one 16-byte load
    def tiny():
        s = torch.cuda.current_stream().cuda_stream
        for i in range(64):
            _lib.check(h.nsv_stream_read(buf.data_ptr() + i * 4096, 16, 1, sink.data_ptr(), s), "stream")
    out["one_load_kernel_us"] = round(_graph_us(tiny, 64, steps=20), 2)
    del buf
    torch.cuda.empty_cache()
    return out


STAMP_POINTS = ["entry", "metadata back", "first tile landed", "key loop done (wave 0)", "waves merged",
                "arrival counted", "split merge done", "every wave's key loop done", "O rows in LDS"]


def stamp_timeline(wl: "Workload", split: int, replays: int = 10) -> dict:
    """Per-workgroup clock stamps of the verify-attention kernel (the stamped
    library, NSV_STAMP_LIB=1), timed like the metric: the 28-call step is
    captured as a hipGraph and replayed.  Every time is taken from the call's
    earliest workgroup entry, in microseconds (the clock ticks every 10 ns).
    Reported per point: the median over the workgroups that reached it, and
    the median over calls of the call's latest workgroup there; and the
    timeline of each call's critical workgroup (the one that finished last),
    median over calls.  Also whether every split of a (sequence, kv head)
    pair ran on one XCD."""
    from naivllm_amd import _lib
    from naivllm_amd.layers.attention import verify_attention_plan

    h = _lib.lib()
    wgs_max, slots = 4096, 16
    calls = wl.layers
    npts = len(STAMP_POINTS)
    buf = torch.zeros(calls * wgs_max * slots, dtype=torch.int64, device=wl.q.device)
    rc = h.nsv_stamp_configure(buf.data_ptr(), calls)
    if rc != 0:
        raise SystemExit("--stamps needs libnaivspec_stamp.so (python -m naivllm_amd.build --stamp)")
    for _ in range(2):
        wl.step(split)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        wl.step(split)
    every = [[] for _ in range(npts)]
    latest = [[] for _ in range(npts)]
    critical = [[] for _ in range(npts)]
    same_xcd = True
    kind, splits = verify_attention_plan(wl.B, wl.H, wl.Hkv, wl.D, wl.bs, wl.max_blocks, wl.rows, torch.bfloat16)
    P8 = (wl.B * wl.Hkv + 7) // 8
    for _ in range(replays):
        buf.zero_()
        graph.replay()
        torch.cuda.synchronize()
        st = buf.view(calls, wgs_max, slots).cpu().numpy()
        for c in range(calls):
            used = np.nonzero(st[c, :, 0] > 0)[0]
            t = st[c][used][:, :npts].astype(np.float64)
            t0 = t[:, 0].min()
            rel = np.where(t > 0, (t - t0) * 0.01, np.nan)
            for i in range(npts):
                v = rel[:, i]
                v = v[~np.isnan(v)]
                if v.size:
                    every[i].extend(v.tolist())
                    latest[i].append(float(v.max()))
            crit = int(np.nanargmax(np.nanmax(rel, axis=1)))
            for i in range(npts):
                if not np.isnan(rel[crit, i]):
                    critical[i].append(float(rel[crit, i]))
            if kind == "key-split":
                xcd = st[c, :, slots - 1]
                groups = {}
                for wg in used:
                    pair = ((wg >> 3) % P8) * 8 + (wg & 7)
                    groups.setdefault(pair, set()).add(int(xcd[wg]))
                same_xcd &= all(len(v) == 1 for v in groups.values())
    h.nsv_stamp_configure(None, 0)
    med = lambda v: round(float(np.median(v)), 2)  # noqa: E731
    out = {"kernel": kind, "splits": splits, "calls": calls * replays, "points_us": {}, "critical_workgroup_us": {}}
    for i, name in enumerate(STAMP_POINTS):
        if every[i]:
            out["points_us"][name] = {"median": med(every[i]), "latest_per_call": med(latest[i])}
        if critical[i]:
            out["critical_workgroup_us"][name] = med(critical[i])
    out["pair_splits_on_one_xcd"] = bool(same_xcd)
    return out


def config4_line(seed: int, steps: int = 20) -> dict:
    """BASELINE config 4 beside the metric's workload: verify attention at the
    Qwen3-8B layer shape (B=16, 32Q/8KV heads, d=128, bf16, 256-token pages,
    contexts uniform in [16k, 32k], K=8), the two rotating pools of
    1,700 pages (1.8 GB each, K and V) far past the Infinity Cache; timed like
    the metric (a hipGraph of one call per pool, HIP events around the
    replays), with its own load-only floor and stream ceilings."""
    wl = Workload(4, 2, seed, torch.device("cuda:0"))
    us = _graph_us(lambda: wl.step(0), wl.layers, steps=steps)
    gbs = wl.bytes / us / 1e3
    tflops = wl.flops / us / 1e6
    out = {"workload": wl.name, "context_lens_sum": int(sum(wl.ctx)), "us_per_call": round(us, 3),
           "bytes_per_call": wl.bytes, "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
           "mfma_tflops": round(tflops, 2), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5),
           "traffic": measured_traffic(4), "ceiling": ceilings(wl)}
    c = out["ceiling"]
    c["kernel_vs_load_floor"] = round(c["load_floor_us"] / us, 4)
    c["kernel_vs_stream"] = round(c["stream_us"] / us, 4)
    del wl
    torch.cuda.empty_cache()
    return out


def rejection_sampling(seed: int = 2, sets: int = 8) -> dict:
    """BASELINE config 2's rejection sampling on the GPU: B = 8, K = 8 model
    drafts per sequence over V = 151936, bf16 draft logits ~ N(0, 2^2) and
    target = draft + 0.5 N(0, 1) (the 9th target row its own N(0, 2^2)),
    drafts sampled from the draft distribution, seeded uniforms and
    exponential noise, T = 1 (nsv_accept_stochastic: min(1, p_t/p_d)
    acceptance with residual resampling).  ``sets`` distinct input sets
    (8 x 51 MB, past the 256 MB Infinity Cache) rotate through a hipGraph
    of one call per set.  Also the greedy acceptance (argmax walk) of the
    same target rows.  Algorithmic bytes per call: the target rows
    (72 x V x 2), the draft rows (64 x V x 2), each sequence's noise row
    (V x 2), uniforms, drafts and outputs."""
    from naivllm_amd.spec_engine.rejection_sampler import accept_greedy, accept_stochastic

    B, K, V = 8, 8, 151936
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    ins = []
    for _ in range(sets):
        draft = (torch.randn(B, K, V, generator=g, device=dev) * 2.0)
        target = torch.empty(B, K + 1, V, device=dev)
        target[:, :K] = draft + 0.5 * torch.randn(B, K, V, generator=g, device=dev)
        target[:, K] = torch.randn(B, V, generator=g, device=dev) * 2.0
        pd = torch.softmax(draft, -1)
        drafts = torch.multinomial(pd.view(-1, V), 1, generator=g).view(B, K).to(torch.int32)
        ins.append(dict(target=target.to(torch.bfloat16).view(B * (K + 1), V).contiguous(),
                        draft=draft.to(torch.bfloat16).view(B * K, V).contiguous(), drafts=drafts,
                        uniforms=torch.rand(B, K, generator=g, device=dev),
                        noise=torch.empty(B, V, device=dev).exponential_(1, generator=g).to(torch.bfloat16)))
        del draft, target, pd
    nd = torch.full((B,), K, dtype=torch.int32, device=dev)
    temp = torch.ones(B, dtype=torch.float32, device=dev)
    out_t = torch.empty(B, K + 1, dtype=torch.int32, device=dev)
    out_n = torch.empty(B, dtype=torch.int32, device=dev)

    def stoch_step():
        for x in ins:
            accept_stochastic(x["target"], x["drafts"], nd, temp, x["noise"], uniforms=x["uniforms"],
                              draft_logits=x["draft"], target_seq_stride=K + 1, draft_seq_stride=K,
                              draft_row_stride=1, out_tokens=out_t, out_len=out_n)

    def greedy_step():
        for x in ins:
            accept_greedy(x["target"], x["drafts"], nd, K + 1, out_tokens=out_t, out_len=out_n)

    margins = _decision_margins(ins, nd, temp, out_t, out_n)
    st_us = _graph_us(stoch_step, sets, steps=20)
    gr_us = _graph_us(greedy_step, sets, steps=20)
    st_bytes = B * (K + 1) * V * 2 + B * K * V * 2 + B * V * 2 + B * K * 4 * 2 + B * 4 + B * (K + 2) * 4 + B * 4
    gr_bytes = B * (K + 1) * V * 2 + B * K * 4 + B * 4 + B * (K + 2) * 4
    del ins
    torch.cuda.empty_cache()
    return {"stochastic": {"us_per_call": round(st_us, 3), "bytes_per_call": st_bytes,
                           "GBs": round(st_bytes / st_us / 1e3, 1),
                           "frac": round(st_bytes / st_us / 1e3 / HBM_PEAK_GBS, 4)},
            "greedy": {"us_per_call": round(gr_us, 3), "bytes_per_call": gr_bytes,
                       "GBs": round(gr_bytes / gr_us / 1e3, 1),
                       "frac": round(gr_bytes / gr_us / 1e3 / HBM_PEAK_GBS, 4)},
            "decision_margins": margins,
            "workload": "config 2 acceptance: B=8, K=8 model drafts, V=151936, bf16 logits, T=1, "
                        f"{sets} rotating input sets"}


def _bf16_round_margin(p: torch.Tensor) -> torch.Tensor:
    """Relative distance of fp64 values p > 0 to the nearest bf16 rounding
    boundary (a midpoint between neighbouring bf16 values): how far an error
    in p may go before its bf16 rounding changes."""
    e = torch.floor(torch.log2(p))
    ulp = torch.exp2(e - 7)
    r = p / ulp  # in [128, 256)
    return (torch.abs(r - torch.floor(r) - 0.5) * ulp) / p


def _decision_margins(ins, nd, temp, out_t, out_n) -> dict:
    """How close config 2's acceptance decisions came to flipping, from the
    same inputs the kernel consumed (torch on the GPU, fp64): for every
    decided draft (the accepted prefix and the first rejection) the margin
    |u - min(1, p_t/p_d)| against the ratio's bf16 ulp, and the relative
    distance of p_t and p_d (exact softmax values) to a bf16 rounding
    boundary; for every sampled row the relative gap between the two
    largest p / q (the multinomial's argmax).  A decision whose margin is
    inside these bands is one that a different softmax reduction order (the
    reference's fp32 torch softmax against this library's exact-then-rounded
    contract) could decide otherwise."""
    from naivllm_amd.spec_engine.rejection_sampler import accept_stochastic

    B, K = nd.shape[0], int(nd[0])
    n_dec, n_band = 0, 0
    min_abs, min_round, min_gap = float("inf"), float("inf"), float("inf")
    for x in ins:
        accept_stochastic(x["target"], x["drafts"], nd, temp, x["noise"], uniforms=x["uniforms"],
                          draft_logits=x["draft"], target_seq_stride=K + 1, draft_seq_stride=K, draft_row_stride=1,
                          out_tokens=out_t, out_len=out_n)
        V = x["target"].shape[-1]
        pt = torch.softmax(x["target"].view(B, K + 1, V).double(), -1)
        pd = torch.softmax(x["draft"].view(B, K, V).double(), -1)
        lens = out_n.tolist()
        for b in range(B):
            acc = lens[b] - 1  # drafts accepted
            for i in range(min(acc + 1, K)):
                d = int(x["drafts"][b, i])
                a, c = pt[b, i, d], pd[b, i, d]
                ab, cb = a.to(torch.bfloat16).float(), c.to(torch.bfloat16).float()
                ratio = torch.clamp((ab / torch.clamp(cb, min=1e-20)).to(torch.bfloat16).float(), max=1.0)
                u = float(x["uniforms"][b, i])
                m = abs(u - float(ratio))
                ulp = 2.0 ** (float(torch.floor(torch.log2(ratio))) - 7)
                n_dec += 1
                n_band += int(m < ulp)
                min_abs = min(min_abs, m)
                min_round = min(min_round, float(_bf16_round_margin(torch.stack([a, c])).min()))
            r = min(acc, K)  # the resampled (rejection) or bonus row
            if acc < K:
                prob = torch.clamp(pt[b, r] - pd[b, r], min=0)
                prob = prob / prob.sum()
            else:
                prob = pt[b, r]
            top = torch.topk(prob / x["noise"][b].double(), 2).values
            min_gap = min(min_gap, float((top[0] - top[1]) / top[0]))
    return {"decisions": n_dec, "min_abs_margin": min_abs, "within_one_bf16_ulp_of_ratio": n_band,
            "min_rel_distance_to_bf16_rounding": min_round, "samples": len(ins) * B,
            "min_rel_top2_gap_of_sample": min_gap}


def copy_probe(mib: int) -> None:
    """Five plain device-to-device copies of ``mib`` MiB (reads and writes
    exactly that many bytes each): the reference point for the HBM traffic
    counters of the verify-attention kernel."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "copies": 5}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--split", type=int, default=0, help="keys per workgroup split (0 = automatic)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ceiling", action="store_true",
                    help="run only the load-only ceilings of the workload (for a rocprofv3 trace) and exit")
    ap.add_argument("--accept", action="store_true",
                    help="run only the config-2 acceptance timings (for a rocprofv3 trace) and exit")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-3 end-to-end round measurement")
    ap.add_argument("--no-cascade", action="store_true",
                    help="skip the config-5 measurement (Qwen3-0.6B drafter feeding Qwen3-8B, hybrid, T=1)")
    ap.add_argument("--stamps", action="store_true",
                    help="load libnaivspec_stamp.so, print the kernel's per-workgroup timeline of the workload "
                         "(medians over workgroups, graph-replayed like the metric) and exit")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--cu-intake", action="store_true",
                    help="time contiguous reads by 32-256 workgroups (one per CU): per-CU against chip-wide intake, and exit")
    ap.add_argument("--batch", type=int, default=8,
                    help="sequences of the config-2 workload for --stamps and --ceiling (1: the b1 round's attention shape)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run only a plain device copy of this many MiB (calibrates rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters against a known byte count) and exit")
    args = ap.parse_args()
    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
        return
    if args.batch != 8 and not (args.stamps or args.ceiling):
        raise SystemExit("--batch applies to --stamps and --ceiling only (the metric is quoted at b8)")
    if not 1 <= args.batch <= 64:
        raise SystemExit("--batch must be in [1, 64]")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        raise SystemExit(2)
    if args.stamps:
        os.environ["NSV_STAMP_LIB"] = "1"  # read when the library is first loaded
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.accept:
        print(json.dumps({"rejection_sampling": rejection_sampling()}), flush=True)
        return
    if args.cu_intake:
        print(json.dumps({"cu_intake": cu_intake()}), flush=True)
        return
    wl = Workload(args.config, args.layers, args.seed, dev, batch=args.batch)
    print(f"[bench] workload: {wl.name}; ctx={wl.ctx}", file=sys.stderr, flush=True)
    if args.ceiling:
        print(json.dumps({"ceiling": ceilings(wl)}), flush=True)
        return
    if args.stamps:
        print(json.dumps({"stamps": stamp_timeline(wl, args.split)}), flush=True)
        return
    # One step (every layer's verify-attention call) is captured as a hipGraph
    # and replayed, as the verify round runs it: the timed region holds GPU
    # work only, not Python launch overhead.
    for _ in range(2):
        wl.step(args.split)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        wl.step(args.split)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_total = e0.elapsed_time(e1)
    ms_per_step = ms_total / args.steps
    calls = args.steps * wl.layers
    us_per_call = ms_total * 1e3 / calls
    gbs = wl.bytes / (us_per_call * 1e-6) / 1e9
    tflops = wl.flops / (us_per_call * 1e-6) / 1e12
    print(f"[bench] {calls} calls, {us_per_call:.2f} us/call, {gbs:.1f} GB/s, {tflops:.1f} TFLOP/s",
          file=sys.stderr, flush=True)

    ceil = ceilings(wl)
    print(f"[bench] ceilings: {ceil}", file=sys.stderr, flush=True)
    wl.k_caches, wl.v_caches = [], []  # free the pools before the other measurements
    torch.cuda.empty_cache()
    c4 = None if args.config == 4 else config4_line(args.seed)
    if c4 is not None:
        print(f"[bench] config 4: {c4}", file=sys.stderr, flush=True)
    accept = rejection_sampling()
    print(f"[bench] acceptance: {accept}", file=sys.stderr, flush=True)
    e2e = None if args.no_e2e else e2e_round()
    self_draft = None if args.no_e2e else e2e_self_draft()
    cascade = None if (args.no_e2e or args.no_cascade) else e2e_cascade()
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded page permutation)",
        "config": {"workload": wl.name, "batch": wl.B, "num_heads": wl.H, "num_kv_heads": wl.Hkv,
                   "head_dim": wl.D, "block_size": wl.bs, "K": wl.K, "context_lens": wl.ctx,
                   "layers_per_step": wl.layers, "kv_split_tokens": args.split},
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "us_per_call": round(us_per_call, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.config),
                     "traffic_source": f"profiles/verify_attn_config{args.config}_traffic.md (rocprofv3 FETCH_SIZE "
                                       f"x2 + WRITE_SIZE x1)",
                     "bytes_per_call": wl.bytes, "mfma_tflops": round(tflops, 2),
                     "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)},
        "ceiling": dict(ceil, kernel_vs_load_floor=round(ceil["load_floor_us"] / us_per_call, 4),
                        kernel_vs_stream=round(ceil["stream_us"] / us_per_call, 4)),
        "config4": c4,
        "rejection_sampling": accept,
        "accepted_tok_s": e2e,
        "accepted_tok_s_k8_self_draft": self_draft,
        "cascade_tok_s": cascade,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
