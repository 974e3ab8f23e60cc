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
    def __init__(self, config: int, layers: int, seed: int, device):
        self.config = config
        if config == 2:
            self.B, self.H, self.Hkv, self.D, self.bs, self.K = 8, 16, 8, 128, 256, 8
            self.ctx = synth.config2_ctx_lens(seed, self.B)
            self.layers = layers
            pool_pages = 64
            name = "verify-attention, Qwen3-0.6B layer shape, b8 bf16, L~U[1200,1300], K=8, 28 layers"
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


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "verify_attn_config2_traffic.md")


def measured_traffic(workload_config: int):
    """HBM bytes per verify-attention launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (copy-calibrated), for the config-2
    workload those passes ran; None otherwise."""
    if workload_config != 2 or not os.path.exists(TRAFFIC_PROFILE):
        return None
    for line in open(TRAFFIC_PROFILE):
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


def cpu_baseline(seconds: float) -> dict:
    """The torch-on-CPU restatement of the same verify-attention call
    (config 2 shape, one layer), timed on this host's cores."""
    from oracle import torch_cpu

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    vb_ctx = synth.config2_ctx_lens(2, 8)
    B, H, Hkv, D, bs, rows = 8, 16, 8, 128, 256, 9
    pages = [(c + bs - 1) // bs for c in vb_ctx]
    g = torch.Generator().manual_seed(2)
    nb = sum(pages) + 4
    kc = torch.randn(nb, bs, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B * rows, H, D, generator=g).to(torch.bfloat16)
    bt = torch.full((B, max(pages)), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :pages[b]] = torch.arange(off, off + pages[b], dtype=torch.int32)
        off += pages[b]
    ctx = torch.tensor(vb_ctx)
    cu = torch.arange(0, B * rows + 1, rows, dtype=torch.int32)
    pos = torch.cat([torch.arange(c - rows, c) for c in vb_ctx])
    args = (q, kc, vc, bt, ctx, cu, pos, 1 / np.sqrt(D), H, Hkv)
    torch_cpu.paged_verify_attention(*args)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        torch_cpu.paged_verify_attention(*args)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    nbytes = algorithmic_bytes(vb_ctx, B * rows, H, Hkv, D, 2, max(pages))
    return {"value": round(nbytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} calls of the config-2 verify-attention (b8 bf16, one layer) in {el:.1f} s, "
                      f"torch CPU restatement of layers/attention.py:328-363 on {platform.processor() or 'host'} "
                      f"with {threads} threads"}


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
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-3 end-to-end round measurement")
    ap.add_argument("--no-cascade", action="store_true",
                    help="skip the config-5 measurement (Qwen3-0.6B drafter feeding Qwen3-8B, hybrid, T=1)")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run only a plain device copy of this many MiB (calibrates rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters against a known byte count) and exit")
    args = ap.parse_args()
    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        raise SystemExit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = Workload(args.config, args.layers, args.seed, dev)
    print(f"[bench] workload: {wl.name}; ctx={wl.ctx}", file=sys.stderr, flush=True)
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

    e2e = None if args.no_e2e else e2e_round()
    cascade = None if (args.no_e2e or args.no_cascade) else e2e_cascade()
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
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
                     "traffic_source": "profiles/verify_attn_config2_traffic.md (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1)",
                     "bytes_per_call": wl.bytes, "mfma_tflops": round(tflops, 2),
                     "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)},
        "accepted_tok_s": e2e,
        "cascade_tok_s": cascade,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
