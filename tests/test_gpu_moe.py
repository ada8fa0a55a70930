"""GPU parity of the NVFP4 grouped-expert MoE forward (titan_moe_nvfp4_forward).

Reference: the expert loop of moe.cpp:874-1005 -- per token and selected
expert, NVFP4 GEMVs (fp4.cu:187-252), SwiGLU (activation.cu:17-32), down
GEMV, weighted combine (activation.cu:111-139).  Two checks per case:
  * fp64 of the same math on the oracle's exact dequantized weights (the
    activations rounded to fp16 as they enter the matrix cores);
  * the reference's own fp32 flow composed from the oracle (or_matvec_nvfp4,
    or_swiglu, or_moe_combine), i.e. what the reference would output.
Tolerance: max |out - ref| <= 1e-3 * max |ref| (plus one ulp of out dtype).
"""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import assert_close_out
from oracle import oracle_ctypes as O

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def make_expert_set(E, hidden, inter, rng):
    """Per expert: REF NVFP4 parts, exact dequantized fp64 matrices, TILED device buffers."""
    ex = []
    for _ in range(E):
        mats = {}
        for name, (n, k) in (("gate", (inter, hidden)), ("up", (inter, hidden)),
                             ("down", (hidden, inter))):
            W = rng.normal(0, 0.02, (n, k)).astype(np.float32)
            g = float(np.abs(W).max() / (6.0 * 448.0))
            w, s = O.quantize_nvfp4(W, g)
            deq = np.asarray(O.dequant_nvfp4(w, s, g, n, k), np.float64).reshape(n, k)
            t = tq.repack_host(tq.NVFP4, n, k, w, s, None, 0)
            mats[name] = dict(w=w, s=s, g=g, deq=deq, dev=torch.from_numpy(t).cuda())
        ex.append(mats)
    table = tq.nvfp4_expert_table([(m["gate"]["dev"], m["up"]["dev"], m["down"]["dev"],
                                    m["gate"]["g"], m["up"]["g"], m["down"]["g"]) for m in ex])
    return ex, table


def routing(T, E, k, rng):
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    logits = rng.normal(0, 1, (T, k))
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    return idx, w.astype(np.float32)


def silu64(g):
    return g / (1.0 + np.exp(-g))


def ref_fp64(ex, x16, idx, w, residual, shared, sw):
    T = x16.shape[0]
    out = np.zeros((T, ex[0]["down"]["deq"].shape[0]))
    for t in range(T):
        acc = 0.0
        for j in range(idx.shape[1]):
            m = ex[idx[t, j]]
            g = m["gate"]["deq"] @ x16[t]
            u = m["up"]["deq"] @ x16[t]
            a = silu64(g) * u
            acc = acc + float(w[t, j]) * (m["down"]["deq"] @ a)
        if shared is not None:
            acc = acc + sw * shared[t]
        out[t] = (residual[t] if residual is not None else 0.0) + acc
    return out


def ref_reference_flow(ex, x32, idx, w, residual, shared, sw, hidden, inter):
    """The reference's fp32 kernels in its order (oracle restatements)."""
    T = x32.shape[0]
    out = np.zeros((T, hidden), np.float32)
    for t in range(T):
        ys = []
        for j in range(idx.shape[1]):
            m = ex[idx[t, j]]
            g = O.matvec_nvfp4(m["gate"]["w"], m["gate"]["s"], m["gate"]["g"], x32[t], inter, hidden)
            u = O.matvec_nvfp4(m["up"]["w"], m["up"]["s"], m["up"]["g"], x32[t], inter, hidden)
            a = O.swiglu(g, u)
            ys.append(O.matvec_nvfp4(m["down"]["w"], m["down"]["s"], m["down"]["g"], a, hidden,
                                     inter))
        res = residual[t] if residual is not None else np.zeros(hidden, np.float32)
        o, _ = O.moe_combine(res, np.stack(ys), w[t], shared[t] if shared is not None else None, sw)
        out[t] = o
    return out


@pytest.mark.parametrize("E,hidden,inter,T,k,xdt,odt,extras", [
    (8, 512, 512, 1, 2, "bf16", "f32", False),     # decode, 16-token passes
    (8, 512, 1024, 5, 4, "f16", "bf16", True),
    (8, 1024, 512, 40, 4, "bf16", "f32", True),    # 32-token passes
    (8, 512, 512, 60, 4, "bf16", "f32", True),     # 48-token passes, experts over 48 tokens
    (8, 512, 512, 70, 8, "f32", "f16", False),     # 64-token passes, an expert over 64 tokens
    (16, 512, 512, 3, 2, "bf16", "f32", False),    # most experts idle
])
def test_moe_nvfp4_forward(E, hidden, inter, T, k, xdt, odt, extras, rng):
    ex, table = make_expert_set(E, hidden, inter, rng)
    idx, w = routing(T, E, k, rng)
    x = torch.from_numpy(rng.normal(0, 1, (T, hidden)).astype(np.float32)).to(TDT[xdt])
    x16 = x.float().half().double().numpy()   # what enters the matrix cores
    residual = rng.normal(0, 0.1, (T, hidden)).astype(np.float32) if extras else None
    shared = rng.normal(0, 0.1, (T, hidden)).astype(np.float32) if extras else None
    sw = 0.37 if extras else 0.0
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty(T, hidden, dtype=TDT[odt], device="cuda")
    tq.moe_nvfp4_forward(table, E, hidden, inter, x.cuda(), torch.from_numpy(idx).cuda(),
                         torch.from_numpy(w).cuda(), out, ws,
                         residual=None if residual is None else torch.from_numpy(residual).cuda(),
                         shared=None if shared is None else torch.from_numpy(shared).cuda(),
                         shared_weight=sw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().astype(np.float64)
    want = ref_fp64(ex, x16, idx, w, residual, shared, sw)
    assert_close_out(got, want, odt)
    flow = ref_reference_flow(ex, x.float().numpy(), idx, w, residual, shared, sw, hidden, inter)
    assert_close_out(got, flow.astype(np.float64), odt)


def test_moe_nvfp4_with_gpu_router(rng):
    """topk_batched on the GPU feeding the grouped forward (C4's decode flow)."""
    E, hidden, inter, T, k = 16, 512, 512, 12, 4
    ex, table = make_expert_set(E, hidden, inter, rng)
    logits = torch.from_numpy(rng.normal(0, 1, (T, E)).astype(np.float32)).cuda()
    wd = torch.empty(T, k, device="cuda")
    idd = torch.empty(T, k, dtype=torch.int32, device="cuda")
    tq.moe_topk_batched(logits, wd, idd, k)
    x = torch.from_numpy(rng.normal(0, 1, (T, hidden)).astype(np.float32)).to(torch.bfloat16)
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty(T, hidden, device="cuda")
    tq.moe_nvfp4_forward(table, E, hidden, inter, x.cuda(), idd, wd, out, ws)
    torch.cuda.synchronize()
    want = ref_fp64(ex, x.float().double().numpy(), idd.cpu().numpy(), wd.cpu().numpy(), None,
                    None, 0.0)
    assert_close_out(out.cpu().numpy().astype(np.float64), want, "f32")


def test_moe_nvfp4_rejects_bad_args(rng):
    E, hidden, inter, T, k = 4, 512, 512, 2, 2
    ex, table = make_expert_set(E, hidden, inter, rng)
    x = torch.zeros(T, hidden, device="cuda", dtype=torch.bfloat16)
    idx = torch.zeros(T, k, dtype=torch.int32, device="cuda")
    w = torch.ones(T, k, device="cuda")
    out = torch.empty(T, hidden, device="cuda")
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(tq.TitanError):
        tq.moe_nvfp4_forward(table, E, hidden, inter, x, idx, w, out, small)
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8,
                     device="cuda")
    with pytest.raises(tq.TitanError):   # inter not a multiple of 512
        tq.moe_nvfp4_forward(table, E, hidden, 384, x, idx, w, out, ws)


def test_moe_nvfp4_every_scale_byte(rng):
    """Every E4M3 block-scale byte, NaNs (0x7F / 0xFF -> 0, fp4.cu:173-185)
    and subnormals included, decodes exactly in the grouped GEMM."""
    E, hidden, inter, T, k = 4, 512, 512, 6, 2
    ex = []
    for e in range(E):
        mats = {}
        for name, (n, kk) in (("gate", (inter, hidden)), ("up", (inter, hidden)), ("down", (hidden, inter))):
            w = rng.integers(0, 256, (n, kk // 2), dtype=np.uint8)
            s = ((np.arange(n * (kk // 16)) * 7 + 31 * e) % 256).astype(np.uint8).reshape(n, kk // 16)
            g = 2e-4
            deq = np.asarray(O.dequant_nvfp4(w, s, g, n, kk), np.float64).reshape(n, kk)
            t = tq.repack_host(tq.NVFP4, n, kk, w, s, None, 0)
            mats[name] = dict(w=w, s=s, g=g, deq=deq, dev=torch.from_numpy(t).cuda())
        ex.append(mats)
    assert set(np.unique(np.concatenate([m["gate"]["s"].ravel() for m in ex]))) == set(range(256))
    table = tq.nvfp4_expert_table([(m["gate"]["dev"], m["up"]["dev"], m["down"]["dev"],
                                    m["gate"]["g"], m["up"]["g"], m["down"]["g"]) for m in ex])
    idx, w = routing(T, E, k, rng)
    x = torch.from_numpy(rng.normal(0, 1, (T, hidden)).astype(np.float32)).to(torch.float16)
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8, device="cuda")
    out = torch.empty(T, hidden, device="cuda")
    tq.moe_nvfp4_forward(table, E, hidden, inter, x.cuda(), torch.from_numpy(idx).cuda(),
                         torch.from_numpy(w).cuda(), out, ws)
    torch.cuda.synchronize()
    want = ref_fp64(ex, x.double().numpy(), idx, w, None, None, 0.0)
    assert np.isfinite(out.cpu().numpy()).all()
    assert_close_out(out.cpu().numpy().astype(np.float64), want, "f32")


@pytest.mark.parametrize("T", [64, 1024])
def test_moe_nvfp4_deepseek_size(T):
    """The benchmark layer at its real size (256 experts, top-8, hidden 7168,
    inter 2048, T = 64 decode and T = 1024 prefill tokens with GPU routing;
    T = 1024 runs the 48/64-token passes per expert): sampled tokens against the
    reference's expert loop restated by the oracle (fp4.cu:187-252 GEMVs with
    the activations rounded to fp16 as they enter the matrix cores, SwiGLU,
    the fp16 activation the kernel stores, weighted sum in slot order)."""
    import bench
    gen = torch.Generator(device="cuda").manual_seed(5 + T)
    E, hidden, inter, k = 256, 7168, 2048, 8
    mats, table = bench.make_nvfp4_experts(E, hidden, inter, gen)
    logits = torch.randn(T, E, generator=gen, device="cuda")
    x = torch.randn(T, hidden, generator=gen, device="cuda").to(torch.bfloat16)
    wd = torch.empty(T, k, device="cuda")
    idd = torch.empty(T, k, dtype=torch.int32, device="cuda")
    tq.moe_topk_batched(logits, wd, idd, k)
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8, device="cuda")
    out = torch.empty(T, hidden, device="cuda")
    tq.moe_nvfp4_forward(table, E, hidden, inter, x, idd, wd, out, ws)
    torch.cuda.synchronize()
    g = 0.02 / 448
    idx, w = idd.cpu().numpy(), wd.cpu().numpy()
    x16 = x.float().half().float().cpu().numpy()
    parts = {}

    def ref_parts(e, j, n, kk):
        if (e, j) not in parts:
            t = mats[e][j].cpu().numpy()
            c, s, _ = tq.unpack_host(tq.NVFP4, n, kk, t, np.zeros((n, kk // 2), np.uint8),
                                     np.zeros((n, kk // 16), np.uint8))
            parts[(e, j)] = (c, s)
        return parts[(e, j)]

    # T = 1024: all 256 experts hold tokens; check the first, last and two
    # middle tokens plus the token routed to the most loaded expert
    toks = {0, T // 2 - 1, T - 1}
    if T > 64:
        load = np.bincount(idx.ravel(), minlength=E)
        toks |= {T // 3, int(np.flatnonzero((idx == load.argmax()).any(1))[-1])}
    for t in sorted(toks):
        acc = np.zeros(hidden, np.float64)
        for q in range(k):
            e = int(idx[t, q])
            gw, gs_ = ref_parts(e, 0, inter, hidden)
            uw, us = ref_parts(e, 1, inter, hidden)
            dw, ds = ref_parts(e, 2, hidden, inter)
            gate = O.matvec_nvfp4(gw, gs_, g, x16[t], inter, hidden)
            up = O.matvec_nvfp4(uw, us, g, x16[t], inter, hidden)
            act = O.swiglu(gate, up).astype(np.float16).astype(np.float32)
            acc += float(w[t, q]) * O.matvec_nvfp4(dw, ds, g, act, hidden, inter).astype(np.float64)
        assert_close_out(out[t].cpu().numpy().astype(np.float64), acc, "f32")
