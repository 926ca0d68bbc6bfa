"""The other BASELINE configs, run by `python bench.py --config N` (config 3, the headline
decode step, lives in bench.py). Each returns one JSON-able dict.

1  split-KV decode attention, one op: q [1,16,128], ctx 1024, page 16, 256-page pool,
   seeded randperm block table, both split policies; vs the CPU oracle op.
2  reshape_and_cache + decode attention at B=32, ctx ~ U[128, 4096], 32k-page x 16 pool,
   nondet heuristic vs fixed-256; cache writes checked bit-exact.
4  DVR verify pass on the Qwen3-0.6B shape: G=4 x W=32 over 2048-token prefixes (time per
   pass, graph replay), plus the watched request's SHA-256 across decode batch widths 1/4/8/16.
5  continuous batching: synthetic requests (prompt lognormal median 512 capped at 8192,
   max_new ~ U[64, 512], seeded Gumbel-max at T=0.7, half of them is_deterministic);
   tokens/s in dvr, nondet and batch_invariant modes.
"""

from __future__ import annotations

import gc
import hashlib
import os
import time

import numpy as np
import torch

HQ, HKV, D = 16, 8, 128
HBM_PEAK_GBS = 8000.0


def _time_us(fn, reps=50, warm=5, graph=True):
    """Average device time per call: reps back-to-back calls captured in one HIP graph and
    replayed between two events (host launch cost is not in the number); graph=False times
    eager launches instead."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    g = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    if g is not None:
        g.replay()
    else:
        for _ in range(reps):
            fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps * 1e3


def _paged(num_pages, lens, rng):
    perm = rng.permutation(num_pages)
    idx, off = [], 0
    for L in lens:
        n = -(-L // 16)
        pages = perm[off:off + n]
        off += n
        pos = np.arange(L)
        idx.append(pages[pos // 16] * 16 + pos % 16)
    indptr = np.zeros(len(lens) + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(lens)
    return (torch.from_numpy(np.concatenate(idx).astype(np.int32)).cuda(),
            torch.from_numpy(indptr.astype(np.int32)).cuda())


def _attn_case(q, k, v, indptr, idx, lens):
    """Both split policies as the engine plans them (nondet: the heuristic splits, segment
    size and stage-1 workgroup shape; batch_invariant: fixed 256-token splits; both with the
    heaviest-first workgroup order), timed as the model runs them: the plan once, then
    back-to-back kernel launches."""
    from sid.kernels.decode_attention import (DecodeAttention, plan_variant, segment_tokens,
                                              workgroup_order)
    from sid.kernels.jit import load_ext
    ext = load_ext()
    attn = DecodeAttention(len(lens), HQ, HKV, D, 32, 256, 32768, "cuda")
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    bytes_ = sum(lens) * (HKV * D * 2 * 2 + 4) + 2 * len(lens) * HQ * D * 2
    out = {}
    o = torch.empty_like(q)
    for name, inv in (("nondet", False), ("fixed256", True)):
        geom, variant = plan_variant(lens, max(lens), HKV, attn.cu_count(), 32, inv)
        ns, grid, fixed, seg, slots = attn.plan(seq, max(lens), inv, geometry=geom)
        tok = segment_tokens(lens, len(lens), grid, fixed, seg, slots)
        order = None  # the engine's rule: an order once the busy segments fill the CUs
        if int((tok > 0).sum()) >= attn.cu_count():
            order = torch.from_numpy(workgroup_order(tok, attn.cu_count())).cuda()
        fn = lambda: ext.flash_decode_fwd(q, k, v, indptr, idx, ns, grid, fixed, D ** -0.5,
                                          attn.part_o, attn.part_lse, o, segment_size=seg,
                                          grid_slots=slots, variant=variant, wg_order=order)
        us = _time_us(fn)
        out[name] = {"us_per_call": round(us, 2), "GB_s": round(bytes_ / us / 1e3, 1),
                     "frac_of_hbm_peak": round(bytes_ / us / 1e3 / HBM_PEAK_GBS, 4),
                     "grid_splits": grid, "segment_tokens": seg, "grid_slots": slots,
                     "stage1_variant": variant}
    return out, attn, seq, bytes_


def _cpu_attention(q, k, v, indptr, idx, min_seconds):
    """The CPU oracle (oracle/attention.py decode_attention_ref) on the same inputs, repeated
    for at least min_seconds; -> (us per call, reference output)."""
    from oracle.attention import decode_attention_ref
    from bench import host_threads
    torch.set_num_threads(host_threads())
    qc, kc, vc, ic, pc = q.cpu(), k.cpu(), v.cpu(), idx.cpu(), indptr.cpu()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < min_seconds or n < 2:
        ref = decode_attention_ref(qc, kc, vc, pc, ic, D ** -0.5)
        n += 1
    return (time.perf_counter() - t0) / n * 1e6, ref, n


def _line(metric, value, unit, higher, workload, roof, cpu, extra):
    from bench import cpu_model, host_threads
    out = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": 50,
           "warmup": 5, "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic: N(0,1) q/K/V, seeded page-shuffled block tables",
           "config": {"workload": workload}, "roofline": roof,
           "cpu_baseline": dict(cpu, cores=host_threads(), kind="port",
                                host_cpus=os.cpu_count(), cpu_model=cpu_model())}
    out.update(extra)
    return out


def _roof(bytes_, us, kernel):
    gbs = bytes_ / us / 1e3
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
            "avg_launch_us": round(us, 2), "bytes_per_launch": int(bytes_)}


def config1(args):
    g = torch.Generator(device="cuda").manual_seed(1)
    q = torch.randn(1, HQ, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(4096, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(4096, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    idx, indptr = _paged(256, [1024], np.random.default_rng(1))
    res, attn, seq, bytes_ = _attn_case(q, k, v, indptr, idx, [1024])
    cpu_us, ref, n = _cpu_attention(q, k, v, indptr, idx, 2.0)
    o = attn.forward(q, k, v, indptr, idx, seq, 1024, D ** -0.5, False)
    err = (o.float().cpu() - ref).abs().max().item()
    us = res["nondet"]["us_per_call"]
    return _line("decode attention op latency, B=1 ctx 1024 page 16 (config 1)", us, "us", False,
                 "split-KV decode attention, one request of 1024 tokens in 16-token pages of a "
                 "256-page shuffled pool, nondet split plan (the reference's heuristic: 32 splits "
                 "of 32 tokens)",
                 _roof(bytes_, us, f"decode_stage1_kernel (variant {res['nondet']['stage1_variant']}) + decode_stage2_kernel"),
                 {"value": round(cpu_us, 1), "unit": "us",
                  "sample": f"oracle.attention.decode_attention_ref on the same inputs, {n} calls"},
                 {"policies": res, "max_abs_err_vs_oracle": err,
                  "note": "4 MiB of K/V: two launches whose fixed latency dominates"})


def config2(args):
    rng = np.random.default_rng(2)
    lens = rng.integers(128, 4097, size=32).tolist()
    g = torch.Generator(device="cuda").manual_seed(2)
    slots = 32768 * 16
    k = torch.randn(slots, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(slots, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    q = torch.randn(32, HQ, D, device="cuda", generator=g).to(torch.bfloat16)
    idx, indptr = _paged(32768, lens, rng)
    new_slots = idx[indptr[1:].long() - 1].long()
    kn = torch.randn(32, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    vn = torch.randn(32, HKV, D, device="cuda", generator=g).to(torch.bfloat16)
    from sid.kernels.jit import load_ext
    ext = load_ext()
    us_cache = _time_us(lambda: ext.reshape_and_cache(kn, vn, k, v, new_slots))
    exact = bool(torch.equal(k[new_slots], kn) and torch.equal(v[new_slots], vn))
    res, attn, seq, bytes_ = _attn_case(q, k, v, indptr, idx, lens)
    cpu_us, ref, n = _cpu_attention(q, k, v, indptr, idx, 3.0)
    o = attn.forward(q, k, v, indptr, idx, seq, max(lens), D ** -0.5, False)
    err = (o.float().cpu() - ref).abs().max().item()
    us = res["nondet"]["us_per_call"]
    return _line("cache write + decode attention, B=32 ctx U[128,4096] (config 2)",
                 res["nondet"]["GB_s"], "GB/s", True,
                 "reshape_and_cache of 32 new K/V rows into a 32k-page x 16 pool, then split-KV "
                 f"decode attention over sum(ctx) = {sum(lens)} tokens in shuffled pages, nondet "
                 "plan (the fixed-256 policy beside it in `policies`)",
                 _roof(bytes_, us, f"decode_stage1_kernel (variant {res['nondet']['stage1_variant']}) + decode_stage2_kernel"),
                 {"value": round(bytes_ / cpu_us / 1e3, 2), "unit": "GB/s",
                  "sample": f"oracle.attention.decode_attention_ref on the same batch, {n} calls, "
                            f"{cpu_us / 1e3:.1f} ms each"},
                 {"policies": res, "max_abs_err_vs_oracle": err, "sum_ctx": int(sum(lens)),
                  "reshape_and_cache": {"us_per_call": round(us_cache, 2), "bit_exact": exact,
                                        "bytes": 32 * HKV * D * 2 * 2 * 2}})


def _engine(mode, layers=None, pool=None, max_reqs=64, seq=4096, batch=64):
    from sid.config import EngineConfig, Mode
    from sid.engine.engine import Engine
    cfg = EngineConfig(mode=Mode(mode), kv_pool_tokens=pool or 400_000, max_reqs=max_reqs,
                       max_seq_len=seq, max_decode_batch=batch, num_layers=layers, seed=0)
    return Engine(cfg)


def config4(args):
    from sid.config import SamplingParams
    eng = _engine("dvr", pool=200_000, max_reqs=40, seq=4096, batch=32)
    vocab = eng.runner.mcfg.vocab_size
    g = torch.Generator().manual_seed(4)
    prompt = lambda n: torch.randint(0, vocab, (n,), generator=g).tolist()
    watched = prompt(2048)
    fillers = [prompt(int(x)) for x in torch.randint(64, 2048, (15,), generator=g)]
    hashes, stats, t_gen = {}, {}, 0.0
    for width in (() if getattr(args, "verify_only", False) else (1, 4, 8, 16)):
        comp = [watched] + fillers[:width - 1]
        params = [SamplingParams(max_new_tokens=96, temperature=0.0, is_deterministic=True,
                                 ignore_eos=True) for _ in comp]
        t0 = time.perf_counter()
        out = eng.generate(comp, params)
        t_gen += time.perf_counter() - t0
        w = out[0]
        hashes[width] = hashlib.sha256(str(w.token_ids).encode()).hexdigest()[:16]
        stats[width] = {"windows": w.num_windows, "rollbacks": w.num_rollbacks}
    # time one verify pass in isolation: G=4 requests with 2048-token prefixes
    from sid.engine.request import RequestState
    runner, ver = eng.runner, eng.verifier
    reqs = []
    for i in range(4):
        rid = eng.add_request(prompt_ids=prompt(2048),
                              params=SamplingParams(max_new_tokens=200, is_deterministic=True,
                                                    ignore_eos=True))
        reqs.append(rid)
    # admit + prefill, then decode 40 tokens without verifying
    new = eng.scheduler.admit()
    for grp in eng.scheduler.prefill_groups(new):
        eng._run_prefill(grp)
    for _ in range(40):
        eng._run_decode(eng.scheduler.decode_reqs())
    group = eng.scheduler.decode_reqs()[:4]
    fb, meta = ver.build_verify_batch(group)
    runner.tag_verify(fb)

    def one():
        runner.step(fb)
    us = _time_us(one, reps=20, warm=3, graph=False)  # runner.step replays its own graph
    # Algorithmic bytes of a pass: every weight once (28 layers + the tied lm_head) and each
    # sequence's K/V rows once per layer (2 x 8 heads x 128 x 2 B per token).
    mcfg = runner.mcfg
    w_bytes = sum(t.numel() * t.element_size() for lw in runner.model.w["layers"]
                  for k_, t in lw.items()) + runner.model.w["lm_head"].numel() * 2
    kv_tokens = int(fb.kv_indptr[-1].item())
    kv_bytes = mcfg.num_layers * kv_tokens * mcfg.num_kv_heads * mcfg.head_dim * 2 * 2
    pass_bytes = w_bytes + kv_bytes
    return {"metric": "DVR verify pass (G=4 x W=32 over 2048-token prefixes) (config 4)",
            "value": round(us / 1e3, 3), "unit": "ms/pass", "higher_is_better": False,
            "roofline": {"bound": "hbm", "achieved": round(pass_bytes / us / 1e3, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pass_bytes / us / 1e3 / HBM_PEAK_GBS, 4),
                         "traffic": None, "kernel": "whole verify pass (native executor)",
                         "bytes_per_launch": int(pass_bytes), "weight_bytes": int(w_bytes),
                         "kv_bytes": int(kv_bytes)},
            "verify_tokens_per_s": round(128 / (us * 1e-6), 1),
            "sha256_watched_by_decode_width": hashes,
            "sha256_identical": (len(set(hashes.values())) == 1) if hashes else None,
            "watched_windows_rollbacks": stats,
            "generate_wall_s": round(t_gen, 2)}


def config5(args):
    from sid.config import SamplingParams
    n = args.stress_requests
    rng = np.random.default_rng(5)
    plen = np.minimum(np.maximum(rng.lognormal(np.log(512), 0.8, n).astype(int), 1), 8192)
    max_new = rng.integers(64, 513, n)
    det = rng.random(n) < 0.5
    prompts = [rng.integers(0, 151936, int(p)).tolist() for p in plen]
    results = {}
    for mode in ("nondet", "dvr", "batch_invariant"):
        # 600k-token pool (69 GB for 28 layers): admission reserves prompt + max_new per
        # request, so at most ~60 of the longest requests, and far more typical ones, fit.
        eng = _engine(mode, pool=600_000, max_reqs=260, seq=9000, batch=256)
        params = [SamplingParams(max_new_tokens=int(m), temperature=0.7, top_p=1.0, seed=i,
                                 is_deterministic=bool(d), ignore_eos=True)
                  for i, (m, d) in enumerate(zip(max_new, det))]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outs = eng.generate(prompts, params)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        toks = sum(len(o.token_ids) for o in outs)
        results[mode] = {"tokens_per_s": round(toks / dt, 1), "wall_s": round(dt, 2),
                         "generated_tokens": toks,
                         "rollbacks": sum(o.num_rollbacks for o in outs)}
        del eng
        gc.collect()
        torch.cuda.empty_cache()
    return {"metric": f"continuous batching, {n} requests, T=0.7 (config 5)",
            "value": results["dvr"]["tokens_per_s"], "unit": "tokens/s", "higher_is_better": True,
            "modes": results,
            "workload": {"prompt_median": int(np.median(plen)), "prompt_max": int(plen.max()),
                         "max_new_mean": float(max_new.mean()), "deterministic_frac": float(det.mean())}}


def run(args):
    return {1: config1, 2: config2, 4: config4, 5: config5}[args.config](args)
