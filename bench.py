"""Headline benchmark: one decode step of a random-init Qwen3-0.6B-shape model (28 layers,
hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072, vocab 151936, tied embeddings) at batch
64 with 2048-token contexts, on one MI355X.

A step is one iteration of the decode token loop: build the decode batch (host + one device
kernel), the 28-layer forward (every op a HIP kernel), greedy sampling, tokens back to the
host. The request state is rolled back after each step so every timed step has identical
work (context 2049). Prints one JSON line with:
  value        decode tokens/s of the whole step
  roofline     the decode-attention op (stage 1 + its merge pass; dominant: ~93% of the
               step's bytes), its average duration measured with HIP events on the launch
               stream, algorithmic bytes per call (K + V rows read + kv_indices + q + o) /
               duration, vs 8 TB/s
  cpu_baseline the CPU oracle (fp32 torch restatement of the step) on a bounded sample
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "deterministic-inference_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=2048)
    ap.add_argument("--mode", default="nondet", choices=["nondet", "dvr", "batch_invariant"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--attn-reps", type=int, default=4)
    ap.add_argument("--eager", action="store_true", help="no HIP graphs (launch every kernel)")
    ap.add_argument("--sync-steps", action="store_true",
                    help="time one synchronous step at a time (no overlapped launch)")
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5],
                    help="BASELINE config: 3 (default) = full decode step; 1 = decode attention op; "
                         "2 = cache write + decode attention at B=32; 4 = DVR verify pass; "
                         "5 = continuous-batching stress")
    ap.add_argument("--stress-requests", type=int, default=512)
    ap.add_argument("--headline-only", action="store_true",
                    help="config 3 only: skip the other BASELINE configs' figures that the "
                         "default run attaches under other_configs")
    ap.add_argument("--verify-only", action="store_true",
                    help="config 4: time the verify pass alone (skip the decode-width token "
                         "comparison), e.g. for a kernel profile of the pass")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one 256 MiB device-to-device copy (known bytes) so that "
                         "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE readings can be scaled")
    return ap.parse_args()


class DecodeWorkload:
    """64 running requests with 2048-token prefixes whose KV is synthetic (N(0,1) bf16 in
    page-shuffled slots); each decode step feeds one token per request at position 2048."""

    def __init__(self, batch, context, mode, seed=0, graphs=True):
        import torch
        from sid.config import EngineConfig, Mode, SamplingParams
        from sid.engine.model_runner import ModelRunner
        from sid.engine.request import Request

        self.torch = torch
        pool = batch * (context + 16) + 4096
        self.cfg = EngineConfig(mode=Mode(mode), kv_pool_tokens=pool, max_reqs=batch + 2,
                                max_seq_len=context + 64, max_decode_batch=batch, seed=seed,
                                use_graphs=graphs)
        self.runner = ModelRunner(self.cfg, "cuda")
        kv = self.kv = self.runner.kv_cache
        g = torch.Generator(device="cuda").manual_seed(seed + 1)
        for pool_t in kv.k_pools + kv.v_pools:
            pool_t.copy_(torch.randn(pool_t.shape, generator=g, device="cuda").to(pool_t.dtype))
        # pages scattered over the pool (page size 16), as after a long run of requests
        kv.scatter_free_pages(seed)
        vocab = self.runner.mcfg.vocab_size
        gen = torch.Generator().manual_seed(seed + 2)
        self.reqs = []
        for i in range(batch):
            r = Request(i, torch.randint(0, vocab, (context,), generator=gen).tolist(),
                        SamplingParams(max_new_tokens=1 << 20, ignore_eos=True),
                        self.runner.mcfg.eos_token_ids)
            r.req_row = kv.open_row()
            kv.grow(r.req_row, context)
            r.output_ids.append(int(torch.randint(0, vocab, (1,), generator=gen)))
            self.reqs.append(r)
        kv.sync_rows([r.req_row for r in self.reqs])
        self.context = context
        self.invariant = self.cfg.mode == Mode.BATCH_INVARIANT

    def build(self):
        return self.runner.prepare_decode(self.reqs, self.invariant)

    def step(self):
        fb = self.build()
        toks = self.runner.step(fb).tolist()
        self.rollback()
        return toks

    def rollback(self, extra: int = 0):
        """Back to context + extra positions per request: a page the step opened beyond
        them goes back to the top of the free stack, so the next step takes the same one
        (identical work)."""
        for r in self.reqs:
            self.kv.shrink(r.req_row, self.context + extra)


def time_steps(wl, steps, warmup, pipelined=True):
    """Seconds per decode step. pipelined: step k+1 is launched before step k's tokens are
    read back, as the engine's overlapped decode runs (EngineConfig.overlap_decode): it
    feeds step k's tokens, gathered on the device, one position further on (context
    2048 + 2); the state is rolled back after each readback, so every step does the same
    work. Otherwise one synchronous step at a time (context 2048 + 1)."""
    torch = wl.torch
    if not pipelined:
        for _ in range(warmup):
            wl.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            wl.step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps
    host = [torch.empty(len(wl.reqs), dtype=torch.int64, pin_memory=True) for _ in range(2)]
    turn = [0]
    import numpy as np
    rows = np.arange(len(wl.reqs), dtype=np.int64)

    def launch(prev=None):
        # As Engine._launch_decode: each request continues from its row of the step still
        # in flight, whose token is gathered on the device (position one further on).
        if prev is None:
            fb = wl.build()
        else:
            fb = wl.runner.prepare_decode(wl.reqs, wl.invariant, prev_rows=rows,
                                          prev_tokens=prev[3])
        tok = wl.runner.step(fb)
        h = host[turn[0]]
        turn[0] ^= 1
        h.copy_(tok, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        return fb, h, ev, tok

    def finish(step):
        fb, h, ev, _ = step
        ev.synchronize()
        toks = h.tolist()
        # same positions next time; a step launched after the first feeds the previous
        # step's token at position context + 1, whose page stays held
        wl.rollback(extra=1)
        return toks

    def run(n):
        prev = launch()
        for _ in range(n - 1):
            nxt = launch(prev)
            finish(prev)
            prev = nxt
        finish(prev)

    run(max(warmup, 1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(steps)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def attention_roofline(wl, reps):
    """Average duration of the decode-attention launch at this step's real shape, HIP events
    on torch's current stream (the launch stream), over reps x 28 layer pools."""
    torch = wl.torch
    fb = wl.build()
    fb.build_indices()
    mcfg = wl.runner.mcfg
    attn = wl.runner.decode_attn
    q = torch.randn(len(wl.reqs), mcfg.num_q_heads, mcfg.head_dim, device="cuda").to(torch.bfloat16)
    scale = mcfg.head_dim ** -0.5
    # warm
    for layer in range(mcfg.num_layers):
        kp, vp = wl.kv.layer(layer)
        attn.forward(q, kp, vp, fb.kv_indptr, fb.kv_indices, fb.seq_lens, fb.max_seq_len, scale,
                     wl.invariant, policy_batch=fb.real_rows, variant=fb.decode_variant,
                     geometry=fb.decode_geometry, wg_order=fb.decode_wg_order)
    torch.cuda.synchronize()
    # One event pair around reps x 28 back-to-back launches on the launch stream: the
    # average is the kernel's steady-state duration (launch overhead overlaps execution).
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    launches = 0
    for _ in range(reps):
        for layer in range(mcfg.num_layers):
            kp, vp = wl.kv.layer(layer)
            attn.forward(q, kp, vp, fb.kv_indptr, fb.kv_indices, fb.seq_lens, fb.max_seq_len,
                         scale, wl.invariant, policy_batch=fb.real_rows,
                         variant=fb.decode_variant, geometry=fb.decode_geometry,
                         wg_order=fb.decode_wg_order)
            launches += 1
    end.record()
    torch.cuda.synchronize()
    avg_ms = start.elapsed_time(end) / launches
    rows = int(fb.kv_indptr[-1].item())
    b = len(wl.reqs)
    bytes_launch = (rows * mcfg.num_kv_heads * mcfg.head_dim * 2 * 2   # K + V rows
                    + rows * 4                                           # kv_indices
                    + 2 * b * mcfg.num_q_heads * mcfg.head_dim * 2)      # q in, o out
    wl.rollback()
    achieved = bytes_launch / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": f"decode_stage1_kernel (workgroup shape {VARIANT_NAMES[fb.decode_variant]}) "
                      "+ decode_stage2_fixed_kernel (all-heads segments of <= 256 tokens, then the "
                      "in-order merge)",
            "avg_launch_us": round(avg_ms * 1e3, 2), "bytes_per_launch": bytes_launch,
            "launches_timed": launches}


VARIANT_NAMES = {0: "4 waves x 4 tokens", 1: "4 waves x 1 token", 2: "8 waves x 2 tokens",
                 3: "4 waves x 2 tokens"}

TRAFFIC_FILE = ROOT / "profiles" / "decode_attention_b64_ctx2048_traffic.json"


def measured_traffic():
    """HBM bytes per call of decode attention (both stages) from the committed rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE runs (scaled by the copy calibration), or None."""
    try:
        return json.loads(TRAFFIC_FILE.read_text())["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(wl, min_seconds=10.0, max_reps=12):
    """The CPU oracle (oracle/qwen3.py) on the same decode batch: whole 28-layer steps,
    repeated until at least min_seconds of CPU time have been measured. Only two layers'
    weights and KV are copied to the host; layer i uses pair i % 2 (the arithmetic per layer
    does not depend on the values, so this is the full step's work at 1/14 of the host
    memory)."""
    import torch
    from oracle.qwen3 import forward_ref

    threads = host_threads()
    torch.set_num_threads(threads)
    fb = wl.build()
    fb.build_indices()
    mcfg = wl.runner.mcfg
    n_layers = mcfg.num_layers
    w = wl.runner.model.w
    two = [{k: v.cpu() for k, v in w["layers"][i].items()} for i in range(2)]
    wc = {"embed": w["embed"].cpu(), "norm": w["norm"].cpu(), "lm_head": w["embed"].cpu(),
          "layers": [two[i % 2] for i in range(n_layers)]}
    used = fb.kv_indices.long()
    rows = used.numel()
    kp2 = [wl.kv.k_pools[i][used].cpu() for i in range(2)]
    vp2 = [wl.kv.v_pools[i][used].cpu() for i in range(2)]
    kp = [kp2[i % 2] for i in range(n_layers)]
    vp = [vp2[i % 2] for i in range(n_layers)]
    indptr = fb.kv_indptr.cpu()
    batch = {"mode": "decode", "input_ids": fb.input_ids.cpu(), "positions": fb.positions.cpu(),
             "out_slots": (indptr[1:] - 1).long(), "kv_indptr": indptr,
             "kv_indices": torch.arange(rows, dtype=torch.int32),
             "sample_indices": torch.arange(len(wl.reqs))}
    wl.rollback()

    forward_ref(wc, mcfg, kp, vp, batch, layers=1)  # warm
    times = []
    while (sum(times) < min_seconds or len(times) < 2) and len(times) < max_reps:
        t0 = time.perf_counter()
        forward_ref(wc, mcfg, kp, vp, batch)
        times.append(time.perf_counter() - t0)
    step = sum(times) / len(times)
    return {"value": round(len(wl.reqs) / step, 3), "unit": "tokens/s", "cores": threads,
            "kind": "port", "host_cpus": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": (f"scaled run of oracle/qwen3.py forward_ref: whole {n_layers}-layer "
                       f"decode steps on the same B={len(wl.reqs)} x ctx {rows // len(wl.reqs)} "
                       f"batch (fp32 arithmetic on bf16 data), with 2 layers' weights and KV "
                       f"copied to the host and reused by all {n_layers} layers (same "
                       f"arithmetic, 1/14 of the host memory); {len(times)} steps in "
                       f"{sum(times):.1f} s, {step:.2f} s per step, on {threads} threads "
                       f"(every CPU this process may run on)")}


def host_threads() -> int:
    """CPUs this process may run on (its affinity mask: the box's CPU share), which is what
    the CPU baseline uses; os.cpu_count() is reported beside it."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def gemm_report(wl):
    """The decode step's non-attention kernels at its real shape (M = batch rows) with their
    weights coming from HBM: the decode chain of every layer in the step's order (input norm
    + qkv + q/k-norm + RoPE + KV write; o + residual; post-attention norm + gate_up + SwiGLU;
    down + residual) over all 28 layers' packed weights, 880 MB, more than the 256 MB
    last-level cache holds, captured in one HIP graph and timed with HIP events around a
    replay. A kernel's figure is the chain's time minus the time of the same chain without
    it, per layer: its in-chain cost, launch boundary included. The lm_head (311 MB, also
    larger than the cache) is timed alone, with its greedy argmax finalize. MFMA rate is
    against the bf16 dense peak, weight-read rate against HBM; at M = 64 these kernels are
    bound by latency, not by either."""
    torch = wl.torch
    from sid.kernels.matmul_persistent import linear_argmax
    from sid.kernels.ops import linear_residual, rmsnorm_linear_silu_mul, rmsnorm_qkv_post
    model = wl.runner.model
    cfg = model.cfg
    w = model.w
    layers = w["layers"]
    packed = model._packed_weights()
    m = len(wl.reqs)
    g = torch.Generator(device="cuda").manual_seed(7)
    xs = {k: torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
          for k in (2048, 3072)}
    residual = torch.randn(m, 1024, device="cuda", generator=g).to(torch.bfloat16)
    r32 = torch.randn(m, 1024, device="cuda", generator=g)
    r32_in = r32.clone()
    pos = torch.arange(m, device="cuda") + 2048
    slots = torch.arange(m, device="cuda")
    k_pool = torch.zeros(m, cfg.num_kv_heads, cfg.head_dim, device="cuda", dtype=torch.bfloat16)
    v_pool = torch.zeros_like(k_pool)
    eps = cfg.rms_norm_eps
    ops = {
        "qkv (norm + q/k-norm + RoPE + KV write)": lambda lw, pw: rmsnorm_qkv_post(
            r32_in, lw["input_ln"], eps, pw["qkv"], lw["q_norm"], lw["k_norm"], pos,
            model.rope.cos_sin, slots, k_pool, v_pool, cfg.num_q_heads),
        "o (+ residual)": lambda lw, pw: linear_residual(xs[2048], pw["o"], residual, r32),
        "gate_up (norm + SwiGLU)": lambda lw, pw: rmsnorm_linear_silu_mul(
            r32_in, lw["post_ln"], eps, pw["gate_up"]),
        "down (+ residual)": lambda lw, pw: linear_residual(xs[3072], pw["down"], residual, r32),
    }
    weights = dict(zip(ops, ("qkv", "o", "gate_up", "down")))

    def timed(fn, reps=1):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(3):
            start.record()
            graph.replay()
            end.record()
            torch.cuda.synchronize()
            best = min(best, start.elapsed_time(end) * 1e3)
        del graph
        return best / reps

    def chain(skip=None):
        def run():
            for lw, pw in zip(layers, packed):
                for name, op in ops.items():
                    if name != skip:
                        op(lw, pw)
        return timed(run)

    full = chain()
    out = {}
    for name in ops:
        us = (full - chain(skip=name)) / len(layers)
        out[name] = (layers[0][weights[name]].shape, us)
    lm = w["lm_head"]
    x1024 = torch.randn(m, 1024, device="cuda", generator=g).to(torch.bfloat16)
    out["lm_head+argmax"] = (lm.shape, timed(lambda: linear_argmax(x1024, lm), reps=20))
    shapes = {}
    for name, ((n, k), us) in out.items():
        flops = 2 * m * n * k
        shapes[name] = {"m": m, "n": n, "k": k, "us": round(us, 2),
                        "tflops": round(flops / us / 1e6, 1),
                        "mfma_frac": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4),
                        "weight_GBps": round(n * k * 2 / us / 1e3, 1),
                        "hbm_frac": round(n * k * 2 / us / 1e3 / HBM_PEAK_GBS, 4)}
    return {"peak_bf16_tflops": MFMA_BF16_PEAK_TFLOPS, "peak_hbm_GBps": HBM_PEAK_GBS,
            "chain_us_per_layer": round(full / len(layers), 2),
            "note": "weights from HBM: the 28 layers' decode chains in step order (880 MB of "
                    "packed weights per pass); per-kernel figures are in-chain costs (chain "
                    "minus chain without it), launch boundaries included",
            "shapes": shapes}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the decode path is single-GPU, as in "
              "the reference); --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.config != 3:
        import bench_configs
        print(json.dumps(bench_configs.run(args)), flush=True)
        return
    wl = DecodeWorkload(args.batch, args.context, args.mode, graphs=not args.eager)
    if args.copy_calib:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    sec = time_steps(wl, args.steps, args.warmup, pipelined=not (args.sync_steps or args.eager))
    roof = attention_roofline(wl, args.attn_reps)
    gemms = gemm_report(wl)
    base = None if args.no_cpu_baseline else cpu_baseline(wl)
    b = args.batch
    out = {
        "metric": "decode tokens/s, Qwen3-0.6B shape bs=64; decode-attn HBM GB/s (% of peak)",
        "value": round(b / sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights ~N(0,0.02), random token ids, N(0,1) KV prefixes",
        "config": {"workload": f"Qwen3-0.6B-shape decode step, batch {b}, context "
                               f"{args.context}+1, greedy, {args.mode} split policy, "
                               f"{'eager launches' if args.eager else 'HIP graph replay'}"
                               f"{'' if (args.sync_steps or args.eager) else ', next step launched before the readback and fed its tokens on the device (overlapped decode; those steps run at context 2048+2)'}",
                   "batch": b, "context": args.context, "layers": wl.runner.mcfg.num_layers,
                   "mode": args.mode},
        "roofline": roof,
        "gemms": gemms,
        "cpu_baseline": base,
    }
    if not args.headline_only:
        # The other BASELINE configs, measured in the same run (each its own workload, after
        # the headline's is freed): 1 and 2 decode-attention ops with rooflines and CPU
        # baselines, 4 the DVR verify pass, 5 continuous batching in the three modes.
        import gc
        import bench_configs
        del wl
        gc.collect()
        torch.cuda.empty_cache()
        others = {}
        for n in (1, 2, 4, 5):
            args.config = n
            others[str(n)] = bench_configs.run(args)
            gc.collect()
            torch.cuda.empty_cache()
        args.config = 3
        out["other_configs"] = others
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
