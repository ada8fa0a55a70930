"""HIP-graph capture of the entry points: they issue only kernels on the
caller's stream (no allocation, no memset, no host synchronisation), so a
captured sequence replays to the eager result.  Every replay is checked
bit-for-bit against the eager run, with the program's own eager work and a
synchronisation between replays."""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import make_weights
from gpu_util import upload
from test_gpu_moe import make_expert_set

pytestmark = pytest.mark.gpu


def replay_check(run, outs, replays=3):
    """run(): issues the work on the current stream into `outs`.  Eager
    result first, then capture, then `replays` replays with unrelated eager
    work (and a rerun of the eager path into scratch) between them."""
    run()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        run()  # warm-up on the capture stream
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.synchronize()
    junk = torch.randn(1 << 20, device="cuda")
    for rep in range(replays):
        for o in outs:
            o.fill_(float("nan") if o.is_floating_point() else -1)
        junk.mul_(1.0001).add_(1.0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o.view(torch.uint8), w.view(torch.uint8)), (rep, i)


@pytest.mark.parametrize("M", [1, 16])
def test_graph_qgemm_batched(M, rng):
    """The batched GEMV (M = 1) and the token-tiled GEMM (M = 16), INT4 TILED."""
    shapes = [(64, 1024), (32, 2048), (48, 1024)]
    Ws, Xs, Ys = [], [], []
    for rows, cols in shapes:
        Ws.append(upload(make_weights("int4", rows, cols, rng), tq.LAYOUT_TILED))
        Xs.append(torch.from_numpy(rng.normal(0, 1, (M, cols)).astype(np.float32)).half().cuda())
        Ys.append(torch.empty(M, rows, dtype=torch.float16, device="cuda"))
    # one argument block per stream: the capture stream binds its own
    calls = {}

    def run():
        st = torch.cuda.current_stream()
        key = st.cuda_stream
        if key not in calls:
            calls[key] = tq.PreparedBatch(Ws, Xs, Ys, stream=st)
        calls[key]()

    replay_check(run, Ys)


def test_graph_fp8_quantize_and_gemm(rng):
    M, N, K = 256, 384, 512
    x = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    W = torch.from_numpy(rng.normal(0, 0.02, (N, K)).astype(np.float32)).cuda()
    sw = (W.abs().amax(1) / 448.0).float()
    wq = (W / sw[:, None]).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    sa = torch.empty(M, device="cuda")
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")

    def run():
        tq.fp8_quantize_rows(x, xq, sa)
        tq.fp8_gemm(xq, sa, wq, sw, out)

    replay_check(run, [xq, sa, out])


def test_graph_moe_router_and_forward(rng):
    E, hidden, inter, T, k = 8, 512, 512, 12, 2
    ex, table = make_expert_set(E, hidden, inter, rng)
    logits = torch.from_numpy(rng.normal(0, 1, (T, E)).astype(np.float32)).cuda()
    wd = torch.empty(T, k, device="cuda")
    idd = torch.empty(T, k, dtype=torch.int32, device="cuda")
    x = torch.from_numpy(rng.normal(0, 1, (T, hidden)).astype(np.float32)).to(torch.bfloat16).cuda()
    ws = torch.empty(tq.moe_nvfp4_workspace_bytes(T, k, E, hidden, inter), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty(T, hidden, device="cuda")

    def run():
        tq.moe_topk_batched(logits, wd, idd, k)
        tq.moe_nvfp4_forward(table, E, hidden, inter, x, idd, wd, out, ws)

    replay_check(run, [wd, idd, out])
