"""HIP graph capture of the SFA forward and backward: replays against eager.

The library launches only kernels on the caller's stream (no memsets, host
copies or synchronisation), so a step can be captured into a HIP graph
(``torch.cuda.CUDAGraph``) and replayed.  Each test captures one call,
replays it several times with unrelated eager work and synchronisations
between the replays, and checks every replay bit for bit against the eager
call on the same inputs (every output here is deterministic).

Covered: the decode-shape forward through the C-ABI with a caller
workspace (token splits and the combine kernel), the same through
``dsa_sfa_fwd_noalloc`` (its fixed scratch array), and the backward through
the Python API (workspace allocated from the graph's pool during capture).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

INT64_MAX = 9223372036854775807
BF = torch.bfloat16


def _decode_inputs(B=4, N1=128, D=512, K=2048, ctx=4096, page=64, seed=5):
    g = torch.Generator(device="cuda").manual_seed(seed)
    nblk = B * ctx // page
    t = {
        "cache": torch.randn(nblk, page, 1, D, generator=g, device="cuda").to(BF),
        "cache_r": torch.randn(nblk, page, 1, 64, generator=g, device="cuda").to(BF),
        "q": torch.randn(B, 1, N1, D, generator=g, device="cuda").to(BF),
        "qr": torch.randn(B, 1, N1, 64, generator=g, device="cuda").to(BF),
        "bt": torch.randperm(nblk, generator=g, device="cuda").to(torch.int32).reshape(B, ctx // page),
        "si": torch.stack([torch.randperm(ctx, generator=g, device="cuda")[:K] for _ in range(B)])
        .to(torch.int32).reshape(B, 1, 1, K).contiguous(),
        "act_k": torch.full((B,), ctx, dtype=torch.int32, device="cuda"),
    }
    return t, (B, N1, D, K, ctx, page, nblk)


def _fwd_call(lib, L, t, dims, outs, noalloc, ws=None, ws_bytes=0):
    B, N1, D, K, ctx, page, nblk = dims
    out, smax, ssum = outs
    args = [t["q"].data_ptr(), t["qr"].data_ptr(), t["cache"].data_ptr(), t["cache_r"].data_ptr(),
            t["si"].data_ptr(), out.data_ptr(), smax.data_ptr(), ssum.data_ptr(), None, t["act_k"].data_ptr(),
            t["bt"].data_ptr(), B, 1, ctx, N1, D, 64, K, B, nblk * page, ctx // page, page, 1, 0,
            INT64_MAX, INT64_MAX, L.LAYOUT["BSND"], L.LAYOUT["PA_BSND"], L.DTYPE_BF16, 1.0 / np.sqrt(D + 64), 1]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = lib.dsa_sfa_fwd_noalloc(*args, stream)
    else:
        st = lib.dsa_sfa_fwd(*args, ws.data_ptr(), ws_bytes, stream)
    L.check(st, "sfa forward")


def _replays_match(graph, outputs, expected, what, n=4):
    for i in range(n):
        for o in outputs:
            o.fill_(float("nan"))              # eager work between replays
        junk = torch.randn(1 << 20, device="cuda").sum()  # an unrelated reduction
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for j, (o, e) in enumerate(zip(outputs, expected)):
            assert torch.equal(o, e), f"{what}: replay {i}: output {j} differs from the eager call"


@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
def test_graph_decode_forward_replays(noalloc):
    from dsa_triton_ascend_amd import _lib as L
    lib = L.load()
    print(f"[graph] decode forward noalloc={noalloc}", flush=True)
    t, dims = _decode_inputs()
    B, N1, D, K = dims[:4]
    ws_bytes = lib.dsa_sfa_fwd_workspace_size(B, N1, D, K, 1)
    assert ws_bytes > 0, "the shape must take the token-split path"
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    outs = (torch.empty(B, 1, N1, D, dtype=BF, device="cuda"), torch.empty(B, 1, 1, N1, device="cuda"),
            torch.empty(B, 1, 1, N1, device="cuda"))
    _fwd_call(lib, L, t, dims, outs, noalloc, ws, ws_bytes)
    torch.cuda.synchronize()
    expected = [o.clone() for o in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _fwd_call(lib, L, t, dims, outs, noalloc, ws, ws_bytes)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _fwd_call(lib, L, t, dims, outs, noalloc, ws, ws_bytes)
    _replays_match(graph, outs, expected, f"decode forward (noalloc={noalloc})")


def test_graph_backward_replays():
    import dsa_triton_ascend_amd as dsa
    from oracle.sfa import sfa_fwd_bsnd
    from tests.helpers import dev, sfa_inputs, sparse_indices, to_dtype_np
    print("[graph] backward", flush=True)
    B, S1, S2, N1, D, K = 1, 24, 320, 128, 512, 96
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=61)
    do = to_dtype_np(np.random.RandomState(62).randn(B, S1, N1, D).astype(np.float32), BF)
    si = sparse_indices(B, S1, S2, K, 1, 3, seed=63)
    scale = 1.0 / np.sqrt(D + 64)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [S1], [S2], 1, 3, True, "float32", positions="kernel")
    args = [dev(q, BF), dev(k, BF), dev(k, BF), dev(si, torch.int32), dev(do, BF), dev(to_dtype_np(out, BF), BF),
            dev(smax, torch.float32), dev(ssum, torch.float32)]
    kw = dict(scale_value=scale, query_rope=dev(qr, BF), key_rope=dev(kr, BF), sparse_mode=3)
    expected = [r.clone() for r in dsa.sparse_flash_attention_grad_triton(*args, **kw)]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dsa.sparse_flash_attention_grad_triton(*args, **kw)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = dsa.sparse_flash_attention_grad_triton(*args, **kw)
    _replays_match(graph, list(outs), expected, "backward")
