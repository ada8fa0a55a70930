"""Benchmark of the quantized matrix-product path on one MI355X.

Headline: INT4 group-wise (group 128, fp16 scale +
fp16 bias, the reference's layout) decode GEMV over one Llama-3-8B layer --
q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096, down
4096x14336 -- at M = 1 fp16 token, fp32 accumulation, fp16 out, weights in
the gfx950 tiled layout.  One step = one pass over the seven matrices (one
batched launch).  `value` = algorithmic bytes per step / time per step.

Secondary lines (same JSON object, key "secondary"): M = 8 / 32 tokens, the
same layer in Q4_K and Q3_K, the Q4_K 4096^2 GEMV, Q3_K / INT2 Llama-3-70B decode shapes
(configs[4]) and the FP8 prefill GEMMs.

The weight set is replicated so that each step reads a copy that is not in
the 256 MB MALL (Infinity Cache) from the previous steps.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "titan-engine_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
LLAMA8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
LLAMA70B = [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)]
ROTATE_BYTES = 768 << 20  # > 3x the 256 MB MALL


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- synthetic weights
def quant_affine_torch(W, gs, bits):
    """convert_titan.py:43-77 recipe on the GPU (fp32 min/max, RNE codes,
    fp16 scale/bias; column 8j+n in nibble n of word j)."""
    import torch
    N, K = W.shape
    levels = (1 << bits) - 1
    G = W.view(N, K // gs, gs)
    mn = G.amin(-1)
    sc = ((G.amax(-1) - mn) / levels).clamp(min=1e-10)
    q = ((G - mn[..., None]) / sc[..., None]).round().clamp(0, levels).to(torch.int64)
    per = 32 // bits
    q = q.view(N, K // per, per)
    sh = torch.arange(per, device=W.device, dtype=torch.int64) * bits
    packed = (q << sh).sum(-1)
    packed = torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)
    return packed, sc.half(), mn.half()


def make_int4_layer(gen, gs=128, bits=4, shapes=LLAMA8B):
    import numpy as np
    import torch
    import titan_qmm as tq
    fmt = tq.INT4 if bits == 4 else tq.INT2
    out = []
    for name, n, k in shapes:
        W = torch.randn(n, k, generator=gen, device="cuda") * 0.02
        w, s, b = quant_affine_torch(W, gs, bits)
        del W
        t = tq.repack_host(fmt, n, k, w.cpu().numpy(), s.cpu().numpy().view(np.uint16),
                           b.cpu().numpy().view(np.uint16), gs)
        out.append(dict(name=name, rows=n, cols=k, fmt=fmt, gs=gs, tiled=torch.from_numpy(t).cuda(),
                        ref=(w, s, b)))
    return out


def random_kquant(fmt, n, k, gen):
    """Synthetic Q4_K / Q3_K bytes: random codes, valid fp16 d/dmin of the
    size N(0, 0.02) weights produce, random 6-bit sub-scales."""
    import numpy as np
    import torch
    import titan_qmm as tq
    nb = k // 256
    bb = 144 if fmt == tq.Q4_K else 110
    blk = torch.randint(0, 256, (n, nb, bb), generator=gen, device="cuda", dtype=torch.int32)
    blk = blk.to(torch.uint8).cpu().numpy()
    d = np.array([0.06 / 63 if fmt == tq.Q4_K else 0.06 / 31 / 4], np.float16).view(np.uint8)
    if fmt == tq.Q4_K:
        blk[:, :, 0:2] = d
        blk[:, :, 2:4] = d
    else:
        blk[:, :, 108:110] = d
    return blk.reshape(n, nb * bb)


# ---------------------------------------------------------------- timing helpers
def time_launches(fn, steps, warmup):
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fn(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per call


def copies_for(nbytes):
    return max(2, min(64, -(-ROTATE_BYTES // max(nbytes, 1))))


# ---------------------------------------------------------------- headline
def bench_int4_layer(M, steps, warmup, gen):
    import torch
    import titan_qmm as tq
    layer = make_int4_layer(gen)
    wbytes = sum(m["tiled"].numel() for m in layer)
    R = copies_for(wbytes)
    copies = [layer] + [[dict(m, tiled=m["tiled"].clone()) for m in layer] for _ in range(R - 1)]
    Ws = [[tq.QWeight(m["fmt"], tq.LAYOUT_TILED, m["rows"], m["cols"], m["tiled"], group_size=m["gs"])
           for m in c] for c in copies]
    X = {k: torch.randn(M, k, generator=gen, device="cuda").half() for k in (4096, 14336)}
    Xs = [X[m["cols"]] for m in layer]
    Ys = [torch.empty(M, m["rows"], device="cuda", dtype=torch.float16) for m in layer]
    abytes = sum(M * m["cols"] * 2 + M * m["rows"] * 2 for m in layer)
    calls = [tq.PreparedBatch(w, Xs, Ys) for w in Ws]
    ms = time_launches(lambda i: calls[i % R](), steps, warmup)
    total = wbytes + abytes
    # per-launch distribution: an event pair around each of `steps` launches
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for i, (a, b) in enumerate(ev):
        a.record()
        calls[i % R]()
        b.record()
    torch.cuda.synchronize()
    each = sorted(a.elapsed_time(b) for a, b in ev)
    pct = {f"p{q}_us": round(1e3 * each[min(len(each) - 1, int(q / 100 * len(each)))], 2)
           for q in (10, 50, 90)}
    return dict(ms=ms, bytes=total, wbytes=wbytes, gbs=total / ms / 1e6, copies=R, pct=pct,
                layer=layer, flops=2 * M * sum(m["rows"] * m["cols"] for m in layer))


def bench_single(W_list, x, y, steps, warmup, algo_bytes):
    import titan_qmm as tq
    R = len(W_list)
    # arguments bound once per copy: the Python cost of building them per
    # call would exceed the kernel time of the small shapes
    calls = [tq.PreparedBatch([w], [x], [y]) for w in W_list]
    ms = time_launches(lambda i: calls[i % R](), steps, warmup)
    return ms, algo_bytes / ms / 1e6


def bench_kquant(fmt, n, k, M, gen, steps, warmup):
    import torch
    import titan_qmm as tq
    blk = random_kquant(fmt, n, k, gen)
    t = tq.repack_host(fmt, n, k, blk)
    dev = torch.from_numpy(t).cuda()
    R = copies_for(dev.numel())
    Wl = [tq.QWeight(fmt, tq.LAYOUT_TILED, n, k, dev if i == 0 else dev.clone()) for i in range(R)]
    x = torch.randn(M, k, generator=gen, device="cuda").half()
    y = torch.empty(M, n, device="cuda", dtype=torch.float16)
    algo = dev.numel() + M * k * 2 + M * n * 2
    ms, gbs = bench_single(Wl, x, y, steps, warmup, algo)
    del Wl, dev
    return dict(ms=ms, gbs=gbs, bytes=algo, ref=(blk, None, None))


def bench_kquant_layer(fmt, M, gen, steps, warmup):
    """One Llama-3-8B layer (LLAMA8B shapes) of synthetic Q4_K / Q3_K codes in
    one batched launch, as the INT4 headline."""
    import torch
    import titan_qmm as tq
    layer = []
    for name, n, k in LLAMA8B:
        t = torch.from_numpy(tq.repack_host(fmt, n, k, random_kquant(fmt, n, k, gen))).cuda()
        layer.append((n, k, t))
    wbytes = sum(t.numel() for _, _, t in layer)
    R = copies_for(wbytes)
    Ws = [[tq.QWeight(fmt, tq.LAYOUT_TILED, n, k, t if c == 0 else t.clone()) for n, k, t in layer]
          for c in range(R)]
    X = {k: torch.randn(M, k, generator=gen, device="cuda").half() for k in (4096, 14336)}
    Xs = [X[k] for _, k, _ in layer]
    Ys = [torch.empty(M, n, device="cuda", dtype=torch.float16) for n, _, _ in layer]
    total = wbytes + sum(M * k * 2 + M * n * 2 for n, k, _ in layer)
    calls = [tq.PreparedBatch(w, Xs, Ys) for w in Ws]
    ms = time_launches(lambda i: calls[i % R](), steps, warmup)
    del Ws, calls, layer
    return dict(ms=ms, gbs=total / ms / 1e6, bytes=total)


def bench_int2(n, k, M, gen, steps, warmup):
    import torch
    import titan_qmm as tq
    (m,) = make_int4_layer(gen, gs=64, bits=2, shapes=[("w", n, k)])
    R = copies_for(m["tiled"].numel())
    Wl = [tq.QWeight(tq.INT2, tq.LAYOUT_TILED, n, k, m["tiled"] if i == 0 else m["tiled"].clone(),
                     group_size=64) for i in range(R)]
    x = torch.randn(M, k, generator=gen, device="cuda").half()
    y = torch.empty(M, n, device="cuda", dtype=torch.float16)
    algo = m["tiled"].numel() + M * k * 2 + M * n * 2
    ms, gbs = bench_single(Wl, x, y, steps, warmup, algo)
    import numpy as np
    w, s, b = m["ref"]
    ref = (w.cpu().numpy().view(np.uint32), s.cpu().numpy().view(np.uint16),
           b.cpu().numpy().view(np.uint16))
    return dict(ms=ms, gbs=gbs, bytes=algo, ref=ref)


def bench_fp8(M, N, K, gen, steps, warmup):
    import torch
    import titan_qmm as tq
    x = torch.randn(M, K, generator=gen, device="cuda").to(torch.bfloat16)
    W = torch.randn(N, K, generator=gen, device="cuda") * 0.02
    sw = (W.abs().amax(1) / 448.0).float()
    wq = (W / sw[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    del W
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(M, device="cuda")
    out = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)

    def step(i):
        tq.fp8_quantize_rows(x, xq, xs)
        tq.fp8_gemm(xq, xs, wq, sw, out)

    ms = time_launches(step, steps, warmup)
    gemm_ms = time_launches(lambda i: tq.fp8_gemm(xq, xs, wq, sw, out), steps, warmup)
    fl = 2.0 * M * N * K
    host = (xq[:4].cpu().numpy(), xs[:4].cpu().numpy(), wq.cpu().numpy(), sw.cpu().numpy())
    return dict(ms=ms, tflops=fl / ms / 1e9, gemm_ms=gemm_ms, gemm_tflops=fl / gemm_ms / 1e9,
                host=host)


NV_EXPERT_BYTES = 3 * (2048 * 7168 // 2 + 2048 * 7168 // 16 + 4)  # codes + e4m3 + global


def make_nvfp4_experts(E, hidden, inter, gen):
    """Synthetic NVFP4 experts directly in the TILED layout: uniform random
    E2M1 codes and E4M3 block scales in [2^-3, 2^2] (no NaN code), fp32
    global scales; the repack is a byte permutation, so random bytes in the
    tiled layout are a valid repacked tensor."""
    import torch
    import titan_qmm as tq
    mats = []
    for _ in range(E):
        trip = []
        for n, k in ((inter, hidden), (inter, hidden), (hidden, inter)):
            nb = tq.tiled_bytes(tq.NVFP4, n, k)
            t = torch.randint(0, 256, (nb,), generator=gen, device="cuda", dtype=torch.int32)
            t = t.to(torch.uint8)
            code_bytes = n * k // 2
            t[code_bytes:] = torch.randint(0x28, 0x48, (nb - code_bytes,), generator=gen,
                                           device="cuda", dtype=torch.int32).to(torch.uint8)
            trip.append(t)
        mats.append(trip)
    table = tq.nvfp4_expert_table([(g, u, d, 0.02 / 448, 0.02 / 448, 0.02 / 448)
                                   for g, u, d in mats])
    return mats, table


def bench_moe(T, steps, warmup, gen, experts=None):
    """C4: DeepSeek-V3-like NVFP4 MoE layer, 256 experts, top-8, hidden 7168,
    inter 2048, T tokens; one step = GPU top-k routing of N(0,1) logits + the
    grouped-expert forward (permute, gate/up+SwiGLU, down, combine)."""
    import torch
    import titan_qmm as tq
    E, hidden, inter, k = 256, 7168, 2048, 8
    mats, table = experts if experts is not None else make_nvfp4_experts(E, hidden, inter, gen)
    logits = torch.randn(T, E, generator=gen, device="cuda")
    x = torch.randn(T, hidden, generator=gen, device="cuda").to(torch.bfloat16)
    w = torch.empty(T, k, device="cuda")
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    out = torch.empty(T, hidden, device="cuda", dtype=torch.bfloat16)
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8,
                     device="cuda")

    def step(i):
        tq.moe_topk_batched(logits, w, idx, k)
        tq.moe_nvfp4_forward(table, E, hidden, inter, x, idx, w, out, ws)

    ms = time_launches(step, steps, warmup)
    torch.cuda.synchronize()
    route = (idx.cpu().numpy(), w.cpu().numpy(), x.float().cpu().numpy())
    used = int(torch.unique(idx).numel())
    nbytes = used * NV_EXPERT_BYTES + T * hidden * 2 * 2 + T * E * 4
    flops = 2.0 * T * k * 3 * inter * hidden
    return dict(ms=ms, experts_hit=used, bytes=nbytes, gbs=nbytes / ms / 1e6,
                tflops=flops / ms / 1e9, route=route), (mats, table)


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(layer, budget_s=12.0):
    """The reference's own AVX-512 CPU expert-path GEMV (matmul_avx.cpp:54-100,
    built from the reference sources into oracle/_ref) over the same INT4
    layer, one thread as in the reference, repeated for a bounded sample."""
    import numpy as np
    from oracle import oracle_ctypes as O
    R = O.ref_lib()
    host = []
    for m in layer:
        w, s, b = m["ref"]
        host.append((w.cpu().numpy().view(np.uint32), s.cpu().numpy().view(np.uint16),
                     b.cpu().numpy().view(np.uint16), m["rows"], m["cols"]))
    xs = {k: np.random.default_rng(0).normal(0, 1, k).astype(np.float32) for k in (4096, 14336)}
    nbytes = sum(m["tiled"].numel() + m["cols"] * 2 + m["rows"] * 2 for m in layer)
    kind = "reference" if R is not None else "port"
    passes, t0 = 0, time.perf_counter()
    while True:
        for w, s, b, n, k in host:
            if R is not None:
                O.ref_matvec_int4(w, s, b, xs[k], n, k, 128)
            else:
                O.matvec_int4_cpu(w, s, b, xs[k], n, k, 128)
        passes += 1
        el = time.perf_counter() - t0
        if el > budget_s or passes >= 50:
            break
    res = dict(value=round(nbytes * passes / el / 1e9, 3), unit="GB/s", cores=1, kind=kind,
               sample=f"{passes} pass(es) of the 7-matrix Llama-3-8B INT4 g128 layer, M=1 fp32 x, "
                      f"{el:.1f} s, {'AVX-512' if R is not None and R.variant == 'avx512' else 'scalar'} "
                      f"build of matmul_avx.cpp, 1 thread")
    # the same loop shape over all host cores (row-partitioned restatement)
    nth = cpu_threads()
    t0 = time.perf_counter()
    mt_passes = 0
    while True:
        for w, s, b, n, k in host:
            O.lib().or_matvec_int4_cpu_mt(*[O._p(a) for a in (w, s, b, xs[k])],
                                          O._p(np.zeros(n, np.float32)), n, k, 128, nth)
        mt_passes += 1
        el = time.perf_counter() - t0
        if el > budget_s / 2 or mt_passes >= 200:
            break
    mt = dict(value=round(nbytes * mt_passes / el / 1e9, 3), unit="GB/s", cores=nth, kind="port",
              sample=f"{mt_passes} pass(es), rows partitioned over {nth} pthreads")
    return res, mt


def cpu_time(fn, budget_s, max_passes=1000):
    passes, t0 = 0, time.perf_counter()
    while True:
        fn()
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s or passes >= max_passes:
            return passes, el


def cpu_gemv_baseline(fmt, ref, g, gs, rows, cols, nbytes, budget_s=1.0):
    """The matmul_avx.cpp:54-100 loop shape (row-serial, column-ascending,
    one fp32 accumulator) restated for `fmt` by the oracle, one thread: the
    reference has no CPU routine for Q4_K / Q3_K / INT2."""
    import numpy as np
    from oracle import oracle_ctypes as O
    codes, sc, bi = ref
    x = np.random.default_rng(1).normal(0, 1, cols).astype(np.float32)
    passes, el = cpu_time(lambda: O.matvec_fmt_mt(fmt, codes, sc, bi, g, gs, x, rows, cols, 1),
                          budget_s)
    one = dict(value=round(nbytes * passes / el / 1e9, 3), unit="GB/s", cores=1, kind="port",
               sample=f"{passes} pass(es) of the {rows}x{cols} {fmt} GEMV, M=1 fp32 x, "
                      f"{el:.2f} s, oracle restatement of the matmul_avx.cpp loop")
    # the same loop with rows partitioned over the host threads
    # (execute_experts_parallel's thread-per-task model, expert_cpu.cpp:39-102)
    nth = cpu_threads()
    passes, el = cpu_time(lambda: O.matvec_fmt_mt(fmt, codes, sc, bi, g, gs, x, rows, cols, nth),
                          budget_s / 2)
    allc = dict(value=round(nbytes * passes / el / 1e9, 3), unit="GB/s", cores=nth, kind="port",
                sample=f"{passes} pass(es), rows partitioned over {nth} pthreads, {el:.2f} s")
    return one, allc


def cpu_threads():
    """Host threads for the all-cores baselines: every core, at most the 16
    cores a one-GPU box grants this job."""
    return max(1, min(os.cpu_count() or 1, 16))


def cpu_moe_baseline(mats, route, hidden, inter, budget_s=2.0):
    """C4 on the host: per token, its k experts in parallel threads, one
    thread per expert (execute_experts_parallel, expert_cpu.cpp:39-102), each
    gate / up / SwiGLU / down with the oracle's NVFP4 GEMV (fp4.cu:187-238
    loop order); weights read back from the GPU's TILED buffers and unpacked."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    import titan_qmm as tq
    from oracle import oracle_ctypes as O
    idx, wts, x = route
    k = idx.shape[1]
    cache = {}

    def ref_of(e):
        if e not in cache:
            parts = []
            for t, (n, kk) in zip(mats[e], ((inter, hidden), (inter, hidden), (hidden, inter))):
                c, s, _ = tq.unpack_host(tq.NVFP4, n, kk, t.cpu().numpy(),
                                         np.zeros((n, kk // 2), np.uint8),
                                         np.zeros((n, kk // 16), np.uint8))
                parts.append((c, s, n, kk))
            cache[e] = parts
        return cache[e]

    g = 0.02 / 448
    toks = 0

    def expert(e, xt):
        (cg, sg, n, kk), (cu, su, _, _), (cd, sd, nd, kd) = ref_of(e)
        a = O.matvec_nvfp4(cg, sg, g, xt, n, kk)
        u = O.matvec_nvfp4(cu, su, g, xt, n, kk)
        h = (a / (1.0 + np.exp(-a)) * u).astype(np.float32)
        return O.matvec_nvfp4(cd, sd, g, h, nd, kd)

    for e in set(idx[:4].reshape(-1).tolist()):
        ref_of(e)  # unpack outside the timed region
    with ThreadPoolExecutor(max_workers=k) as pool:
        t0 = time.perf_counter()
        while True:
            t = toks % min(4, idx.shape[0])
            ys = list(pool.map(lambda j: expert(int(idx[t, j]), x[t]), range(k)))
            _ = sum(wts[t, j] * ys[j] for j in range(k))
            toks += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    nbytes = toks * k * NV_EXPERT_BYTES
    return dict(value=round(nbytes / el / 1e9, 3), unit="GB/s", cores=k, kind="port",
                ms_per_token=round(1e3 * el / toks, 1),
                sample=f"{toks} token(s), {k} experts each on {k} threads, {el:.2f} s")


def cpu_fp8_baseline(host, N, K, budget_s=1.0):
    """The oracle's scalar FP8 GEMM (e4m3 x e4m3, fp32 accumulate, per-token
    and per-channel scales) on a sample of activation rows, one thread; the
    reference has no FP8 CPU path."""
    from oracle import oracle_ctypes as O
    A, sa, W, sw = host
    rows = 1
    passes, el = cpu_time(lambda: O.gemm_fp8(A[:rows], sa[:rows], W, sw), budget_s, max_passes=50)
    return dict(value=round(2.0 * rows * N * K * passes / el / 1e12, 6), unit="TFLOP/s", cores=1,
                kind="port", sample=f"{passes} pass(es) of {rows} activation row x {N}x{K}, {el:.2f} s")


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


# ---------------------------------------------------------------- HBM traffic
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qgemv_int4_llama8b_m1_traffic.md")
COPY_CALIB_BYTES = 1 << 30


def copy_calibration():
    """A plain device copy of COPY_CALIB_BYTES: its FETCH_SIZE / WRITE_SIZE per
    dispatch is the scale that turns those counters into HBM bytes."""
    import torch
    src = torch.empty(COPY_CALIB_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {COPY_CALIB_BYTES} bytes 5 times")


def traffic_from_profile():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 --pmc summary: the line `traffic_bytes_per_launch: <n>`."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except (OSError, ValueError):
        pass
    return None


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--fp8-only", action="store_true",
                    help="only the two FP8 prefill GEMMs (for counter runs); prints their lines")
    ap.add_argument("--int4-layer-tokens", type=int, default=0,
                    help="only the INT4 8B layer at this token count (for counter runs); prints its line")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calib:
        copy_calibration()
        return
    import titan_qmm as tq
    tq.lib()
    gen = torch.Generator(device="cuda").manual_seed(0)
    K, W = args.steps, args.warmup

    if args.fp8_only:
        lines = []
        for (M, N, Kd) in [(2048, 14336, 4096), (2048, 4096, 14336)]:
            r = bench_fp8(M, N, Kd, gen, K, W)
            lines.append(dict(config=f"FP8 E4M3 GEMM M={M} N={N} K={Kd}", ms=round(r["ms"], 4),
                              gemm_only_TFLOPS=round(r["gemm_tflops"], 1)))
        print(json.dumps(lines))
        return

    if args.int4_layer_tokens > 0:
        M = args.int4_layer_tokens
        r = bench_int4_layer(M, K, W, gen)
        print(json.dumps(dict(config="INT4 g128 Llama-3-8B layer", M=M, ms=round(r["ms"], 4),
                              GBps=round(r["gbs"], 1), frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4))))
        return

    log("headline: INT4 g128 Llama-3-8B layer, M=1")
    h = bench_int4_layer(1, K, W, gen)
    secondary = []
    if not args.headline_only:
        for M in (8, 32):
            r = bench_int4_layer(M, max(20, K // 4), 5, gen)
            secondary.append(dict(config="INT4 g128 Llama-3-8B layer", M=M, ms=round(r["ms"], 4),
                                  GBps=round(r["gbs"], 1), frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4),
                                  TFLOPS=round(r["flops"] / r["ms"] / 1e9, 2)))
            del r
        for fmt, nm in ((tq.Q4_K, "Q4_K"), (tq.Q3_K, "Q3_K")):
            log(f"{nm} Llama-3-8B layer M=1")
            r = bench_kquant_layer(fmt, 1, gen, K, W)
            secondary.append(dict(config=f"{nm} Llama-3-8B layer (q,k,v,o,gate,up,down; synthetic codes)",
                                  M=1, ms=round(r["ms"], 5), GBps=round(r["gbs"], 1),
                                  frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4)))
            torch.cuda.empty_cache()
        log("Q4_K 4096x4096")
        r = bench_kquant(tq.Q4_K, 4096, 4096, 1, gen, K, W)
        secondary.append(dict(config="Q4_K 4096x4096 GEMV (synthetic codes)", M=1,
                              ms=round(r["ms"], 5), GBps=round(r["gbs"], 1),
                              frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4)))
        if not args.no_cpu:
            (secondary[-1]["cpu_baseline"],
             secondary[-1]["cpu_baseline_all_cores"]) = cpu_gemv_baseline("q4k", r["ref"], 0.0, 0, 4096,
                                                                          4096, r["bytes"])
        for M in (1, 4):
            for n, k in LLAMA70B:
                log(f"Q3_K / INT2 {n}x{k} M={M}")
                r = bench_kquant(tq.Q3_K, n, k, M, gen, max(20, K // 2), 5)
                secondary.append(dict(config=f"Q3_K {n}x{k} GEMV (synthetic codes)", M=M,
                                      ms=round(r["ms"], 5), GBps=round(r["gbs"], 1),
                                      frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4)))
                if M == 1 and not args.no_cpu:
                    (secondary[-1]["cpu_baseline"],
                     secondary[-1]["cpu_baseline_all_cores"]) = cpu_gemv_baseline(
                        "q3k", r["ref"], 0.0, 0, n, k, r["bytes"], budget_s=0.5)
                r = bench_int2(n, k, M, gen, max(20, K // 2), 5)
                secondary.append(dict(config=f"INT2 g64 {n}x{k} GEMV", M=M, ms=round(r["ms"], 5),
                                      GBps=round(r["gbs"], 1),
                                      frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4)))
                if M == 1 and not args.no_cpu:
                    (secondary[-1]["cpu_baseline"],
                     secondary[-1]["cpu_baseline_all_cores"]) = cpu_gemv_baseline(
                        "int2", r["ref"], 0.0, 64, n, k, r["bytes"], budget_s=0.5)
                torch.cuda.empty_cache()
        ex = None
        for T in (64, 1024):
            log(f"NVFP4 MoE T={T}")
            r, ex = bench_moe(T, max(20, K // 10), 5, gen, ex)
            secondary.append(dict(config=f"NVFP4 MoE 256 experts top-8 7168/2048 T={T} "
                                         "(synthetic codes)", T=T, ms=round(r["ms"], 4),
                                  experts_hit=r["experts_hit"], GBps=round(r["gbs"], 1),
                                  frac_hbm=round(r["gbs"] / HBM_PEAK_GBS, 4),
                                  TFLOPS=round(r["tflops"], 1)))
            if T == 64 and not args.no_cpu:
                log("NVFP4 MoE CPU baseline")
                secondary[-1]["cpu_baseline"] = cpu_moe_baseline(ex[0], r["route"], 7168, 2048)
        del ex
        torch.cuda.empty_cache()
        for (M, N, Kd) in [(2048, 14336, 4096), (2048, 4096, 14336)]:
            log(f"FP8 GEMM {M}x{N}x{Kd}")
            # steady state: the first launches after the MoE lines run cold
            r = bench_fp8(M, N, Kd, gen, max(50, K // 4), 20)
            secondary.append(dict(config=f"FP8 E4M3 GEMM M={M} N={N} K={Kd} (+act quant)",
                                  ms=round(r["ms"], 4), TFLOPS=round(r["tflops"], 1),
                                  gemm_only_TFLOPS=round(r["gemm_tflops"], 1),
                                  frac_fp8_peak=round(r["gemm_tflops"] / FP8_PEAK_TFLOPS, 4)))
            if not args.no_cpu:
                secondary[-1]["cpu_baseline"] = cpu_fp8_baseline(r["host"], N, Kd)

    cpu, cpu_mt = (None, None)
    if not args.no_cpu:
        log("cpu baseline")
        cpu, cpu_mt = cpu_baseline(h["layer"])
        cpu["cpu_model"] = cpu_model()

    line = {
        "metric": "Q4_K/INT4 decode GEMV GB/s (% of HBM peak); FP8/FP4 GEMM TFLOPS (% peak)",
        "value": round(h["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(h["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic: weights N(0,0.02) quantized on the GPU with the convert_titan.py "
                "INT4 recipe; x ~ N(0,1) fp16",
        "config": {"workload": "INT4 g128 dequant-GEMV, one Llama-3-8B layer (q,k,v,o,gate,up,down), "
                               "M=1, tiled layout, one batched launch per step",
                   "arithmetic": "int4 codes x fp16 activations, fp32 accumulate, fp16 out",
                   "algorithmic_bytes_per_step": h["bytes"], "weight_bytes": h["wbytes"],
                   "weight_copies_rotated": h["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(h["gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(h["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile(), "kernel": "qgemv_kernel (INT4 tiled, MFMA fold)",
                     "algorithmic_bytes_per_launch": h["bytes"],
                     "timing": "torch.cuda.Event pair on the launch stream around all timed launches",
                     "per_launch": dict(h["pct"], note="event pair around each launch, "
                                        "includes the launch gap")},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_mt,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
