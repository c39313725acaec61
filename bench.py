"""Sparse-MLA decode benchmark on one MI355X.

Workload: the 32K-context decode step, B=8 sequences, H=64 heads, latent rows 576 (512 + 64 rope)
in bf16.  Raw latent cache [8, 32768, 576] (window rows), block-4 mean-pooled compressed cache
[8, 8192, 576], fp8-e4m3 indexer keys [8, 8192, 64] with per-row pow2 scales, top-k 2048 plus the
128-row window at position 32767.

One step = indexer score -> exact top-k (+ window ids) -> split-K MFMA attention + LSE merge,
for all 8 sequences; metric value = tokens/s = B * K / (time of K steps).  Inputs are resident in
HBM; R copies of the caches (> 512 MB of distinct rows touched per rotation) are rotated so the
256 MB MALL cannot serve the gather.  The K steps are replayed from HIP graphs.

Also reported:
* roofline of the dominant kernel (the MFMA attention split kernel): algorithmic bytes per launch /
  its average duration, measured with HIP events around graph replays of that kernel alone (one
  launch per rotated cache copy, back to back);
* cpu_baseline: the CPU oracle running the same step on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "deepseek-v4-flash-mlx_amd")
sys.path.insert(0, PKG)

METRIC = "sparse-MLA decode tok/s/GPU @32K ctx top-k 2048; HBM GB/s; prefill MFMA util"
HBM_PEAK_GBS = 8000.0


def algorithmic_attention_bytes(B, H, T, D=576, DV=512, row_bytes=1152):
    """Rows gathered + q read + output written + index list read, per launch."""
    return B * T * row_bytes + B * H * D * 2 + B * H * DV * 2 + B * T * 4


BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA

KERNEL_NAME = "attn_decode_kernel<576>"


def measured_traffic(kernel, workload="decode_32k"):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (both counters scaled by a plain-copy calibration); None when the summary has no such line."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{workload}_hbm_counters.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {kernel} {workload}:"):
                    return int(line.rsplit(":", 1)[1])
    except OSError:
        return None
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--rot", type=int, default=24, help="cache copies rotated across steps")
    ap.add_argument("--kernel-iters", type=int, default=96)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=5, help="CPU baseline: median of this many runs after 1 warm-up")
    ap.add_argument("--rows-per-split", type=int, default=0,
                    help="attention split plan: index-list rows per split, a multiple of 32 (0 = the default plan)")
    ap.add_argument("--decode-path", choices=("lists", "select-in-attn"), default="lists",
                    help="timed decode step: indexer, selection launch, list attention (the default), or "
                         "indexer then smla_decode_attn (the selection inside the attention workgroups)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill MFMA-utilisation leg")
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--no-others", action="store_true", help="skip the other workloads and kernels")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB, 8 times (HBM counter calibration)")
    return ap.parse_args()


def copy_calibration(mib):
    """A plain copy kernel of known size: `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` on this run gives
    the counter reading per byte moved, which scales the same counters read on the attention kernel."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": mib << 20, "launches": 8}), flush=True)


def prefill_measure(dev, reps):
    """Prefill (S=4096 queries, H=64, 576-wide bf16 rows): each query attends its 128-row raw
    window and every causally visible block-4 compressed row.  One attention launch per pass
    (one split per query); MFMA utilisation = algorithmic flops / time / dense bf16 peak."""
    import torch
    from smla import compressor as scomp
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    w = wl.prefill_4k()
    H = w["q"].shape[2]
    q = w["q"].to(dev)
    raw = w["raw"].to(dev)
    comp = scomp.block_mean_pool(raw, 4)
    idx = wl.prefill_indices(4096, ratio=4, window=128, n_raw=4096)
    pairs = int((idx >= 0).sum())                  # (query, row) pairs
    flops = 2.0 * pairs * H * (576 + 512)
    idx = idx[None].to(dev)

    def timed(fn):
        for _ in range(5):  # untimed passes first: the clock settles over the first few
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    # the prefill entry (row sets computed in the kernel, longest lists first) and the same
    # attention over explicit index lists
    implicit = lambda: ssa.prefill_attn(q, raw, comp, None, w["scale"], q_pos0=0, window=128, ratio=4)
    lists = lambda: ssa.sparse_attn_two_source(q, raw, comp, None, idx, w["scale"], dv=512)
    ms, ms_lists = float("inf"), float("inf")
    for _ in range(2):  # alternated, best of two each (the clock settles over the first passes)
        ms = min(ms, timed(implicit))
        ms_lists = min(ms_lists, timed(lists))
    tflops = flops / (ms * 1e-3) / 1e12
    return {"workload": "prefill_4k: S=4096 queries, H=64, raw [4096,576] + mean-pooled [1024,576] bf16, "
                        "window 128 + causal compressed rows (smla_prefill_attn)",
            "ms": round(ms, 4), "flops": flops, "query_row_pairs": pairs, "tflops": round(tflops, 1),
            "mfma_peak_tflops": BF16_PEAK_TFLOPS, "mfma_util": round(tflops / BF16_PEAK_TFLOPS, 4),
            "ms_method": f"the better of two timed rounds of {reps} passes each (5 untimed passes before each)",
            "ms_index_lists": round(ms_lists, 4)}


def _time_ms(fn, reps):
    import torch
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _time_graph_ms(fn, reps, inner=20):
    """GPU time of one call of `fn`: `inner` calls captured in one HIP graph after two eager
    warm-ups, the graph replayed `reps` times between HIP events; host dispatch and the graph
    launch are amortised over inner * reps calls."""
    import torch
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    ms = _time_ms(graph.replay, max(3, reps // inner) if inner > 1 else reps) / inner
    del graph
    torch.cuda.synchronize()
    return ms


def other_workloads(dev, reps):
    """The other decode workloads and the path's remaining kernels, each captured in a HIP graph
    and timed with HIP events over `reps` replays on resident inputs (inputs smaller than the
    256 MB MALL may be served from it on repeats; the block-mean pool's 377 MB, the fp4 keys'
    512 MB and the rotating o_proj weights are not)."""
    import torch
    from smla import compressor as scomp
    from smla import indexer as sidx
    from smla import norm_rope as snr
    from smla import ops
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    res = {}

    # ---- fp32_plumbing: B=1, H=16, fp32 q/rows [4096,576], fp32 indexer keys [4096,64], top-512,
    # the fp32 attention (the vector-ALU kernel: fp32 operands keep the reference's precision)
    w = wl.fp32_plumbing()
    q1, kv1, qi1, ki1, w1 = (w[t].to(dev) for t in ("q", "kv", "q_idx", "k_idx", "w"))

    def run_c1():
        sc = sidx.indexer_score(qi1[None], ki1[None], None, w1[None])
        sel = sidx.topk(sc[0], w["k"])
        return ssa.sparse_attn(q1, kv1, None, sel, w["scale"], dv=w["dv"])
    ms = _time_graph_ms(run_c1, reps)
    gather = w["k"] * 576 * 4 + 16 * 576 * 4 + 16 * 512 * 4 + w["k"] * 4
    res["fp32_plumbing"] = {"workload": "fp32_plumbing: B=1 H=16, fp32 q [16,576] and rows [4096,576], fp32 indexer "
                                        "keys [4096,64] (16 heads), top-512, fp32 attention",
                            "us_per_step": round(ms * 1e3, 3), "gather_bytes": gather,
                            "achieved_gbs": round(gather / (ms * 1e-3) / 1e9, 1)}
    del q1, kv1, qi1, ki1, w1

    # ---- decode_64k: one sequence, 20 consecutive positions 65516..65535; per step: indexer over
    # the (p+1)//4 visible compressed keys, window + top-2048 ids, attention, merge
    w = wl.decode_64k()
    raw = w["raw"].to(dev)
    comp = scomp.block_mean_pool(raw, 4)
    keys, ks = w["k_codes"].to(dev), w["kscale"].to(dev)
    qi, wt, q = w["q_idx"].to(dev), w["w"].to(dev), w["q"].to(dev)
    n_raw, k, win = raw.shape[1], w["k"], w["window"]
    poss = [w["pos0"] + i for i in range(w["steps"])]
    nvis = [torch.tensor([[(p + 1) // 4]], dtype=torch.int32, device=dev) for p in poss]
    posd = [torch.tensor([p], dtype=torch.int32, device=dev) for p in poss]

    def run64():
        for i in range(w["steps"]):
            sc = sidx.indexer_score(qi[i][None, None], keys, ks, wt[i][None, None], nvis[i])
            idx = sidx.select_decode_indices(sc[:, 0], k, posd[i], win, n_raw)
            ssa.sparse_attn_two_source(q[i][None], raw, comp, None, idx[:, None, :], w["scale"], dv=512)
    ms = _time_graph_ms(run64, max(1, reps // 4), inner=1)
    per = ms / w["steps"]
    step_bytes = algorithmic_attention_bytes(1, 64, win + k)
    nk = keys.shape[1]
    idx_bytes = nk * (64 + 4) + nk * 4          # fp8 keys + scales read, scores written
    res["decode_64k"] = {"workload": "decode_64k: B=1 H=64, raw [65536,576] + mean-pooled [16384,576] bf16, fp8 keys "
                                     "[16384,64], 20 steps at positions 65516..65535, top-k 2048 + window 128",
                         "tok_s": round(w["steps"] / (ms * 1e-3), 1), "ms_per_step": round(per, 4),
                         "attention_bytes_per_step": step_bytes, "indexer_bytes_per_step": idx_bytes,
                         "achieved_gbs": round((step_bytes + idx_bytes) / (per * 1e-3) / 1e9, 1),
                         "achieved_gbs_note": "attention + indexer algorithmic bytes over the whole step "
                                              "(indexer, selection, attention, merge): a latency-bound step"}

    # ---- batched_fp8: 64 sequences, e4m3 rows with pow2 scales, 2048 ids each (attention + merge)
    w = wl.batched_fp8()
    qb, codes, scl, idxb = w["q"].to(dev), w["codes"].to(dev), w["scales"].to(dev), w["idx"].to(dev)
    ms = _time_graph_ms(lambda: ssa.sparse_attn_batched(qb, codes, None, idxb, w["scale"], dv=512, kv_scale=scl), reps)
    nsel = int((w["idx"] >= 0).sum())
    fb = nsel * 612 + 64 * 64 * 576 * 2 + 64 * 64 * 512 * 2 + nsel * 4
    res["batched_fp8"] = {"workload": "batched_fp8: B=64 H=64, e4m3 rows (612 B with 9 fp32 pow2 scales), lengths "
                                      "U{2048..16384}, 2048 ids per sequence",
                          "tok_s": round(64 / (ms * 1e-3), 1), "ms": round(ms, 4), "algorithmic_bytes": fb,
                          "achieved_gbs": round(fb / (ms * 1e-3) / 1e9, 1)}
    del qb, codes, scl, idxb

    # ---- kernels of the decode_32k step, at its shapes
    w = wl.decode_32k()
    raw = w["raw"].to(dev)
    qi, keys, ks, wt = w["q_idx"].to(dev), w["k_codes"].to(dev), w["kscale"].to(dev), w["w"].to(dev)
    B, N, Hi, Di = 8, keys.shape[1], qi.shape[2], qi.shape[3]
    ms = _time_graph_ms(lambda: sidx.indexer_score(qi, keys, ks, wt), reps)
    flops = 2.0 * B * N * Hi * Di
    res["indexer_score"] = {"shape": "B=8 Hi=64 Di=64 N=8192, bf16 q x e4m3 keys, fixed-order fp32 fma chains",
                            "us": round(ms * 1e3, 3), "bound": "valu fp32",
                            "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 2), "peak_tflops": 157.3,
                            "hbm_bytes": B * N * (Di + 4) + B * N * 4}
    # the same scores over keys in the indexer compressor's fp4 form (Hadamard + e2m1, ue8m0 per 32)
    from smla import qat as sqat
    kc4, ks4 = sqat.fp4_pack(torch.randn(B, N, Di, device=dev), rotate=True)
    ms = _time_graph_ms(lambda: sidx.indexer_score_fp4(qi, kc4, ks4, ks, wt), reps)
    res["indexer_score_fp4"] = {"shape": "B=8 Hi=64 Di=64 N=8192, bf16 q x fp4 keys (packed e2m1 + ue8m0 per 32), "
                                         "fixed-order fp32 fma chains",
                                "us": round(ms * 1e3, 3), "bound": "valu fp32",
                                "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 2), "peak_tflops": 157.3,
                                "hbm_bytes": B * N * (Di // 2 + Di // 32 + 4) + B * N * 4}
    del kc4, ks4
    sc = sidx.indexer_score(qi, keys, ks, wt)
    pos = torch.full((B,), w["pos"], dtype=torch.int32, device=dev)
    ms = _time_graph_ms(lambda: sidx.select_decode_indices(sc[:, 0], w["k"], pos, w["window"], raw.shape[1]), reps)
    res["select_decode"] = {"shape": "8 rows x 8192 scores, k=2048, window 128 (one launch)",
                            "us": round(ms * 1e3, 3), "bound": "latency (one workgroup per row)"}
    ws = torch.empty(ops.index_decode_workspace(B, 1, N), dtype=torch.uint8, device=dev)
    ms = _time_graph_ms(lambda: sidx.index_decode(qi, keys, ks, wt, None, w["k"], pos, w["window"], raw.shape[1],
                                            workspace=ws), reps)
    res["index_decode"] = {"shape": "B=8 Hi=64 Di=64 N=8192 -> window 128 + top-2048 ids: fixed-order scores "
                                    "on the matrix cores, exact selection (two launches in one call)",
                           "us": round(ms * 1e3, 3)}
    ms = _time_graph_ms(lambda: scomp.block_mean_pool(raw, 4), max(2, reps // 2))
    mb = raw.numel() * 2 + raw.numel() // 4 * 2
    res["block_mean_pool"] = {"shape": "[8,32768,576] bf16 -> [8,8192,576]", "us": round(ms * 1e3, 3),
                              "bytes": mb, "achieved_gbs": round(mb / (ms * 1e-3) / 1e9, 1), "peak_gbs": HBM_PEAK_GBS}
    del raw
    g = torch.Generator().manual_seed(7)
    kvp = torch.randn(1, 4096, 1024, generator=g).to(dev)
    scp = torch.randn(1, 4096, 1024, generator=g).to(dev)
    ape = torch.randn(4, 1024, generator=g).to(dev)
    nw = torch.rand(512, generator=g).to(dev)
    cos_t, sin_t = snr.rope_tables(64, 65536, device=dev)
    ms = _time_graph_ms(lambda: ops.gated_pool_op(kvp, scp, ape, nw, cos_t, sin_t, 4, 64, 1e-6, 1), reps)
    gb = 2 * kvp.numel() * 4 + 1024 * 512 * 4 + 1024 * 32 * 4 * 2
    res["gated_pool"] = {"shape": "kv, score [1,4096,1024] fp32 -> [1,1024,512] (overlap softmax + RMSNorm + RoPE + fp8 sim)",
                         "us": round(ms * 1e3, 3), "bytes": gb, "achieved_gbs": round(gb / (ms * 1e-3) / 1e9, 1)}
    x = torch.randn(8192, 576, generator=g).to(dev)
    ms = _time_graph_ms(lambda: ops.quant_fp8_pow2_op(x), reps)
    qbytes = x.numel() * 4 + x.numel() + x.numel() // 64 * 4
    res["quant_fp8_pow2"] = {"shape": "[8192,576] fp32 -> e4m3 codes + per-64 pow2 scales", "us": round(ms * 1e3, 3),
                             "bytes": qbytes, "achieved_gbs": round(qbytes / (ms * 1e-3) / 1e9, 1)}
    del x
    # indexer keys: 1M rows of 128 (512 MB of fp32, larger than the 256 MB MALL) -> stored fp4 form
    xk = torch.randn(1 << 20, 128, device=dev)
    ms = _time_graph_ms(lambda: ops.rotate_fp4_op(xk, True, True, False, True), max(2, reps // 2))
    kb = xk.numel() * 4 + xk.numel() // 2 + xk.numel() // 32
    res["rotate_fp4"] = {"shape": "[1048576,128] fp32 -> Hadamard + fp4 e2m1 (packed codes + ue8m0 per 32)",
                         "us": round(ms * 1e3, 3), "bytes": kb, "achieved_gbs": round(kb / (ms * 1e-3) / 1e9, 1),
                         "peak_gbs": HBM_PEAK_GBS}
    del xk
    # attention output path of one decode step: 8 tokens, inverse RoPE + o_grouped (wo_a 8x[1024,4096],
    # wo_b [4096,8192], bf16).  Three weight copies (384 MB) rotate so the MALL cannot hold them.
    T, ncopy = 8, 3
    wts = [((torch.randn(8192, 4096, device=dev) * 0.02).to(torch.bfloat16),
            (torch.randn(4096, 8192, device=dev) * 0.02).to(torch.bfloat16)) for _ in range(ncopy)]
    o = torch.randn(T, 64, 512, device=dev).to(torch.bfloat16)
    opos = torch.arange(30000, 30000 + T, dtype=torch.int32, device=dev)
    ct, st_ = snr.rope_tables(64, 65536, device=dev)
    calls = [lambda i=i: ops.o_proj_op(o, opos, ct, st_, wts[i][0], wts[i][1], 8, torch.bfloat16)
             for i in range(ncopy)]
    for c in calls:
        c()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    ms = _time_ms(graph.replay, max(2, reps // 4)) / ncopy
    ob = 2 * 8192 * 4096 * 2 + o.numel() * 2 + T * 8192 * 2 * 2 + T * 4096 * 2
    res["o_proj"] = {"shape": "T=8 tokens: inverse RoPE + o_grouped, wo_a [8192,4096] + wo_b [4096,8192] bf16 "
                              "(two launches; a graph of 3 calls over rotating weight copies, per call)",
                     "us": round(ms * 1e3, 3), "bytes": ob, "achieved_gbs": round(ob / (ms * 1e-3) / 1e9, 1),
                     "peak_gbs": HBM_PEAK_GBS}
    del graph, wts

    # ---- prompt-size projections through the tiled MFMA GEMM (smla_linear beyond 32 token rows):
    # 4096 tokens, bf16 operands; MFMA utilisation against the dense bf16 peak
    gemm = {}
    for name, T, G, N, K, odt in (("q_down", 4096, 1, 1024, 4096, torch.float32),
                                  ("wq_b_wkv", 4096, 1, 8192, 4096, torch.float32),
                                  ("wo_a_grouped", 4096, 8, 1024, 4096, torch.bfloat16),
                                  ("wo_b", 4096, 1, 4096, 8192, torch.bfloat16)):
        x = (torch.randn(T, G * K, device=dev) * 0.1).to(torch.bfloat16)
        wm = (torch.randn(G * N, K, device=dev) * 0.02).to(torch.bfloat16)
        ms = _time_graph_ms(lambda: ops.linear_op(x, wm, G, odt), max(4, reps // 4))
        fl = 2.0 * T * G * N * K
        gemm[name] = {"shape": f"[{T},{G * K}] x [{G * N},{K}]^T" + (f" in {G} groups" if G > 1 else ""),
                      "us": round(ms * 1e3, 2), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                      "mfma_util": round(fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}
        del x, wm
    res["prefill_gemm"] = gemm

    # ---- decode_layer: the whole attention layer for one token (projections, RoPE, fp8 sim, window
    # append, compressor ring, take-all ids, attention, output projection), 8 sequences at position
    # 32767 over filled 32K caches; a graph of 5 steps (each rewrites the same cache rows)
    from smla import engine
    g = torch.Generator(device="cpu").manual_seed(5)
    bf = lambda *s: (torch.randn(*s, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    f32 = lambda *s: (1.0 + 0.1 * torch.randn(*s, generator=g)).to(dev)
    lw = engine.LayerWeights(wq_a=bf(1024, 4096), q_a_norm=f32(1024), wq_b=bf(64 * 512, 1024), wkv=bf(512, 4096),
                             kv_a_norm=f32(512), wo_a=bf(8 * 1024, 4096), wo_b=bf(4096, 8 * 1024), sinks=f32(64),
                             wkv_c=bf(1024, 4096), wgate_c=bf(1024, 4096), ape=f32(4, 1024), norm_c=f32(512))
    B, P = 8, 32768
    layer = engine.DecodeLayer(lw, B, 4, max_pos=P, device=dev)
    layer.raw.normal_(0, 0.5)
    layer.comp.normal_(0, 0.5)
    xn = (torch.randn(B, 4096, generator=g)).to(torch.bfloat16).to(dev)
    pos = torch.full((B,), P - 1, dtype=torch.int32, device=dev)
    ms = _time_graph_ms(lambda: layer.step(xn, pos), reps, inner=5)
    wbytes = sum(t.numel() * t.element_size() for t in (lw.wq_a, lw.wq_b, lw.wkv, lw.wo_a, lw.wo_b, lw.wkv_c,
                                                         lw.wgate_c))
    res["decode_layer"] = {"workload": "decode_layer: one attention layer, B=8 tokens at position 32767, 128-row window "
                                       "ring + 8192 compressed rows (take-all: 128 + 8192 ids), 231 MB of bf16 "
                                       "weights; graph of 5 steps",
                           "us": round(ms * 1e3, 3), "tok_s": round(B / (ms * 1e-3), 1), "weight_bytes": wbytes}
    del layer

    # ---- prefill_layer: the same layer's prompt branch (DecodeLayer.prefill: projections through the
    # tiled GEMM, row epilogues, gated pool into the compressed cache, ring set-up, prompt attention,
    # output projection) for one 4096-token prompt into a fresh layer; best of 3 after 2 untimed runs
    S = 4096
    xp = (torch.randn(1, S, 4096, generator=g)).to(torch.bfloat16).to(dev)
    best = float("inf")
    for rep in range(5):
        player = engine.DecodeLayer(lw, 1, 4, max_pos=S + 64, device=dev)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        player.prefill(xp)
        e1.record()
        torch.cuda.synchronize()
        if rep >= 2:
            best = min(best, e0.elapsed_time(e1))
        del player
    res["prefill_layer"] = {"workload": "prefill_layer: the decode_layer's weights, one 4096-token prompt into a fresh "
                                        "layer (DecodeLayer.prefill), eager launches",
                            "ms": round(best, 4), "tok_s": round(S / (best * 1e-3), 1),
                            "ms_method": "best of 3 after 2 untimed runs"}
    del lw, xp
    return res


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it: the first `model name` line with the cpu family,
    model and stepping numbers (virtual machines often shorten the name to the vendor line), or
    None."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                key, _, val = line.partition(":")
                fields.setdefault(key.strip(), val.strip())
    except OSError:
        return None
    name = fields.get("model name")
    if name is None:
        return None
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_baseline(w, nthreads, reps):
    """Time the oracle on one full decode step (all 8 sequences): C indexer chain + C top-k +
    torch sparse attention, median of `reps` after one warm-up."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import indexer as oidx
    from oracle import sparse_attn as osa
    from oracle import compressor as ocomp
    os.environ["OMP_NUM_THREADS"] = str(nthreads)
    torch.set_num_threads(nthreads)
    B, k, win = w["q"].shape[0], w["k"], w["window"]
    n_raw = w["raw"].shape[1]
    comp = ocomp.mean_pool(w["raw"], 4).to(torch.bfloat16)
    keys = w["k_codes"].view(torch.float8_e4m3fn).float().numpy()
    ks = w["kscale"].numpy()
    qi = w["q_idx"].float().numpy()
    wt = w["w"].numpy()
    raw_f = [w["raw"][b, n_raw - win:].float() for b in range(B)]
    comp_f = [comp[b].float() for b in range(B)]
    qf = w["q"].float()

    def one_step():
        for b in range(B):
            sc = oidx.indexer_score(qi[b], keys[b], ks[b], wt[b])
            sel = oidx.topk(sc, k)[0]
            kv = torch.cat([raw_f[b], comp_f[b][torch.from_numpy(sel).long()]])
            ids = torch.arange(kv.shape[0], dtype=torch.int32)[None]
            osa.sparse_attn(qf[b], kv, None, ids, w["scale"], dv=512)

    one_step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_step()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return med


def _median_time(fn, reps):
    """Median wall time of `reps` calls of fn after one warm-up call."""
    import numpy as np
    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_legs(nthreads, reps):
    """The oracle on the other configurations, on the host's cores (median of `reps` after one
    warm-up each): fp32_plumbing (whole step), prefill_4k (a sample of 8 of its 64 query chunks of
    64, every 8th, extrapolated by query-row pairs), decode_64k (4 of its 20 steps) and batched_fp8
    (all 64 sequences, each sequence's gathered rows dequantised)."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import compressor as ocomp
    from oracle import indexer as oidx
    from oracle import sparse_attn as osa
    from smla import workloads as wl
    torch.set_num_threads(nthreads)
    res = {}

    w = wl.fp32_plumbing()
    qi, ki, wt = w["q_idx"].numpy(), w["k_idx"].numpy(), w["w"].numpy()

    def c1():
        sc = oidx.indexer_score(qi, ki, None, wt)
        sel = oidx.topk(sc, w["k"])
        osa.sparse_attn(w["q"], w["kv"], None, torch.from_numpy(sel), w["scale"], dv=w["dv"])
    t = _median_time(c1, reps)
    res["fp32_plumbing"] = {"ms_per_step": round(t * 1e3, 3), "sample": "the whole step (indexer, top-512, attention)"}

    w = wl.prefill_4k()
    q = w["q"][0].float()
    raw = w["raw"]
    comp = ocomp.mean_pool(raw, 4).to(torch.bfloat16)
    kv = torch.cat([raw[0].float(), comp[0].float()])
    idx = wl.prefill_indices(4096, ratio=4, window=128, n_raw=4096)
    chunks = list(range(0, 64, 8))
    pairs_all = int((idx >= 0).sum())
    pairs_s = sum(int((idx[64 * c:64 * c + 64] >= 0).sum()) for c in chunks)

    def c3():
        for c in chunks:
            osa.sparse_attn(q[64 * c:64 * c + 64], kv, None, idx[64 * c:64 * c + 64], w["scale"], dv=512)
    t = _median_time(c3, reps)
    res["prefill_4k"] = {"ms_sample": round(t * 1e3, 2), "sample_query_row_pairs": pairs_s,
                         "ms_full_extrapolated": round(t * 1e3 * pairs_all / pairs_s, 1),
                         "gflops": round(2.0 * pairs_s * 64 * 1088 / t / 1e9, 1),
                         "sample": "8 of the 64 chunks of 64 queries (every 8th), extrapolated to the whole "
                                   "prompt by query-row pairs"}
    del q, raw, comp, kv

    w = wl.decode_64k()
    comp = ocomp.mean_pool(w["raw"], 4).to(torch.bfloat16)[0].float()
    raw_f = w["raw"][0].float()
    keys = w["k_codes"][0].view(torch.float8_e4m3fn).float().numpy()
    ks = w["kscale"][0].numpy()
    n_raw, win, k = raw_f.shape[0], w["window"], w["k"]

    def c4():
        for i in range(4):
            p = w["pos0"] + i
            nv = (p + 1) // 4
            sc = oidx.indexer_score(w["q_idx"][i].float().numpy()[None], keys, ks, w["w"][i].numpy()[None],
                                    np.array([nv], dtype=np.int32))
            sel = oidx.topk(sc, k, np.array([nv], dtype=np.int32))[0]
            kvb = torch.cat([raw_f[p - win + 1:p + 1], comp[torch.from_numpy(sel[sel >= 0]).long()]])
            osa.sparse_attn(w["q"][i].float(), kvb, None, torch.arange(kvb.shape[0], dtype=torch.int32)[None],
                            w["scale"], dv=512)
    t = _median_time(c4, reps)
    res["decode_64k"] = {"ms_per_step": round(t * 1e3 / 4, 3), "sample": "4 of the 20 steps (indexer over 16384 "
                                                                         "keys, top-2048, attention)"}
    del comp, raw_f, keys

    w = wl.batched_fp8()

    def c5():
        for b in range(w["q"].shape[0]):
            ids = w["idx"][b, 0]
            ids = ids[ids >= 0].long()
            rows = wl.dequant_e4m3(w["codes"][b, ids], w["scales"][b, ids])
            osa.sparse_attn(w["q"][b].float(), rows, None, torch.arange(rows.shape[0], dtype=torch.int32)[None],
                            w["scale"], dv=512)
    t = _median_time(c5, reps)
    res["batched_fp8"] = {"ms_per_step": round(t * 1e3, 2), "tok_s": round(64 / t, 1),
                          "sample": "all 64 sequences (gathered rows dequantised, then attention)"}
    return res


def main():
    args = parse()
    if args.copy_mib:
        copy_calibration(args.copy_mib)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world > 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(sharding across GPUs is designed, not run)"}))
        sys.exit(2)

    import numpy as np
    import torch
    import smla
    from smla import _lib
    from smla import compressor as scomp
    from smla import indexer as sidx
    from smla import ops
    from smla import sparse_attn as ssa
    from smla import workloads as wl

    smla.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print("[bench] generating decode_32k inputs", file=sys.stderr, flush=True)
    w = wl.decode_32k()
    B, k, win = w["q"].shape[0], w["k"], w["window"]
    H = w["q"].shape[2]
    n_raw = w["raw"].shape[1]
    T = win + k

    raw0 = w["raw"].to(dev)
    comp0 = scomp.block_mean_pool(raw0, 4)
    keys0 = w["k_codes"].to(dev)
    ks0 = w["kscale"].to(dev)
    copies = [(raw0, comp0, keys0, ks0)]
    for _ in range(args.rot - 1):
        copies.append(tuple(t.clone() for t in copies[0]))
    q = w["q"].to(dev)
    qi = w["q_idx"].to(dev)
    wt = w["w"].to(dev)
    pos = torch.full((B,), w["pos"], dtype=torch.int32, device=dev)
    print(f"[bench] {args.rot} cache copies resident ({args.rot * sum(t.numel() * t.element_size() for t in copies[0]) / 2**30:.1f} GiB)",
          file=sys.stderr, flush=True)

    ws = torch.empty(ops.index_decode_workspace(B, 1, keys0.shape[1]), dtype=torch.uint8, device=dev)

    wsd = torch.empty(ops.decode_attn_workspace(B, 1, H, 576, 512, win, k), dtype=torch.uint8, device=dev)

    def step_fused(r):
        raw, comp, keys, ks = copies[r]
        sc = sidx.indexer_score(qi, keys, ks, wt)
        return ssa.decode_attn(q, raw, comp, None, sc[:, 0], pos, win, k, w["scale"], dv=512, workspace=wsd)

    def step_lists(r):
        raw, comp, keys, ks = copies[r]
        sc = sidx.indexer_score(qi, keys, ks, wt)
        idx = sidx.select_decode_indices(sc[:, 0], k, pos, win, n_raw)
        return ops.sparse_attn_ex(q, raw, comp, None, None, None, idx[:, None, :], w["scale"], 512,
                                  rows_per_split=args.rows_per_split)

    fused = args.decode_path == "select-in-attn" and args.rows_per_split == 0
    step = step_fused if fused else step_lists

    ref_out = step(0)
    torch.cuda.synchronize()

    # ---- capture R consecutive steps (one per cache copy) into a graph
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for r in range(args.rot):
            step(r)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graphs = {}
    timing = [False]

    def graph_for(nsteps):
        if nsteps not in graphs:
            if timing[0]:
                raise RuntimeError(f"graph of {nsteps} steps was not captured before the timed region")
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                outs = [step(r) for r in range(nsteps)]
            graphs[nsteps] = (g, outs)
        return graphs[nsteps]

    def run_steps(n):
        full, tail = divmod(n, args.rot)
        for _ in range(full):
            graph_for(args.rot)[0].replay()
        if tail:
            graph_for(tail)[0].replay()

    # every graph the warm-up and the timed steps replay is captured here, outside the timed region
    for n in (args.rot, args.warmup % args.rot, args.steps % args.rot):
        if n:
            graph_for(n)
    torch.cuda.synchronize()
    g_full, outs = graph_for(args.rot)
    # every replay must reproduce the eager result (copies hold identical data)
    for rep in range(2):
        g_full.replay()
        torch.cuda.synchronize()
        for o in outs:
            if not torch.equal(o, ref_out):
                raise SystemExit("graph replay differs from the eager step")
    print("[bench] graph replays match the eager step", file=sys.stderr, flush=True)

    run_steps(args.warmup)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    timing[0] = True
    e0.record()
    run_steps(args.steps)
    e1.record()
    torch.cuda.synchronize()
    timing[0] = False
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / args.steps
    tok_s = B * args.steps / (ms / 1000.0)
    print(f"[bench] {args.steps} steps in {ms:.3f} ms", file=sys.stderr, flush=True)

    # ---- dominant kernel: MFMA attention, events around the kernel alone (eager, rotated copies)
    ns, rps, _ = ops.attn_plan(B, 1, H, 576, 512, T, rows_per_split=args.rows_per_split)
    idx_all = []
    for r in range(args.rot):
        raw, comp, keys, ks = copies[r]
        idx_all.append(sidx.index_decode(qi, keys, ks, wt, None, k, pos, win, n_raw, workspace=ws))
    torch.cuda.synchronize()
    # the split kernel alone (phase SMLA_ATTN_SPLIT): a graph of `rot` launches, one per cache copy, on
    # preallocated outputs and workspaces, replayed back to back between two events on the replay stream
    _, _, wsb = ops.attn_plan(B, 1, H, 576, 512, T, rows_per_split=args.rows_per_split)
    k_out = [torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device=dev) for _ in range(args.rot)]
    k_ws = [torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev) for _ in range(args.rot)]

    def split_only(r):
        ops.sparse_attn_ex(q, copies[r][0], copies[r][1], None, None, None, idx_all[r][:, None, :], w["scale"], 512,
                           rows_per_split=args.rows_per_split, phases=_lib.ATTN_SPLIT, out=k_out[r],
                           workspace=k_ws[r])

    for r in range(args.rot):
        split_only(r)
    torch.cuda.synchronize()
    gk = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gk):
        for r in range(args.rot):
            split_only(r)
    gk.replay()
    torch.cuda.synchronize()
    reps = max(1, args.kernel_iters // args.rot)
    ka, kb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ka.record()
    for _ in range(reps):
        gk.replay()
    kb.record()
    torch.cuda.synchronize()
    k_us = 1000.0 * ka.elapsed_time(kb) / (reps * args.rot)
    full_ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    # main + merge, per op (eager)
    full_ev[0].record()
    for i in range(args.kernel_iters):
        r = i % args.rot
        ops.sparse_attn_ex(q, copies[r][0], copies[r][1], None, None, None, idx_all[r][:, None, :], w["scale"], 512,
                           rows_per_split=args.rows_per_split, out=k_out[r], workspace=k_ws[r])
    full_ev[1].record()
    torch.cuda.synchronize()
    attn_op_us = 1000.0 * full_ev[0].elapsed_time(full_ev[1]) / args.kernel_iters

    alg_bytes = algorithmic_attention_bytes(B, H, T)
    achieved = alg_bytes / (k_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(KERNEL_NAME),
                "traffic_source": "profiles/decode_32k_hbm_counters.md (rocprofv3 --pmc, copy-calibrated)",
                "kernel": KERNEL_NAME, "kernel_us": round(k_us, 3),
                "algorithmic_bytes": alg_bytes, "nsplit": ns, "rows_per_split": rps}

    # the other decode-step form, timed the same way (graph replays over the rotated copies); both
    # run the default split plan, so only then are their outputs the same bit for bit
    alt = None
    if args.rows_per_split == 0:
        alt_step = step_lists if fused else step_fused
        g_alt = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_alt):
            alt_outs = [alt_step(r) for r in range(args.rot)]
        g_alt.replay()
        torch.cuda.synchronize()
        if not all(torch.equal(o, ref_out) for o in alt_outs):
            raise SystemExit("the two decode-step forms differ")
        alt_reps = max(1, args.steps // args.rot)
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(alt_reps):
            g_alt.replay()
        eb.record()
        torch.cuda.synchronize()
        alt_us = 1000.0 * ea.elapsed_time(eb) / (alt_reps * args.rot)
        alt = {"decode_path": "lists" if fused else "select-in-attn", "us_per_step": round(alt_us, 3),
               "tok_s": round(B / (alt_us * 1e-6), 1), "output": "bit-identical to the timed step"}

    prefill = None
    if not args.no_prefill:
        print("[bench] prefill leg", file=sys.stderr, flush=True)
        prefill = prefill_measure(dev, args.prefill_reps)

    others = None
    if not args.no_others:
        print("[bench] other workloads and kernels", file=sys.stderr, flush=True)
        others = other_workloads(dev, 10)

    cpu = None
    if not args.no_cpu_baseline:
        ncores = len(os.sched_getaffinity(0))
        print(f"[bench] cpu baseline on {ncores} threads", file=sys.stderr, flush=True)
        med = cpu_baseline(w, ncores, args.cpu_steps)
        cpu = {"value": round(B / med, 2), "unit": "tok/s", "cores": ncores, "kind": "port",
               "cpu_model": _cpu_model(),
               "sample": f"one full decode step (8 sequences: indexer chain + top-k + attention), "
                         f"median of {args.cpu_steps} after 1 warm-up; {med * 1e3:.1f} ms/step"}
        print("[bench] cpu legs of the other configurations", file=sys.stderr, flush=True)
        legs = cpu_legs(ncores, args.cpu_steps)
        for name, leg in legs.items():
            leg.update(cores=ncores, kind="port", median_of=args.cpu_steps)
        if prefill is not None:
            prefill["cpu_baseline"] = legs.pop("prefill_4k")
        if others is not None:
            for name in list(legs):
                if name in others:
                    others[name]["cpu_baseline"] = legs.pop(name)
        if legs:
            cpu["other_configs"] = legs

    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1)*0.05 q/latent rows (bf16), fp8 indexer keys, seed 1",
        "config": {"workload": "decode_32k: B=8 H=64 rows 576 bf16, raw [8,32768,576], mean-pooled "
                               "[8,8192,576], fp8 keys [8,8192,64], top-k 2048 + window 128",
                   "global_batch": B, "seq_len": 32768, "parallelism": "single GPU",
                   "decode_path": "select-in-attn" if fused else "lists"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "other": others,
        "attention_op_us": round(attn_op_us, 3),
        "other_decode_path": alt,
        "rotated_copies": args.rot,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
