"""Outputs the caller did not request, through the C-ABI.

The reference returns zeros for softmax_max / softmax_sum when
return_softmax_lse is off (sparse_flash_attention_triton.py:527, 616-617)
and for the indexer's values when return_value is off.  The library writes
those zeros itself into buffers the caller passes with the flag off, so the
Python API allocates them without a fill.  Each case passes NaN-filled
buffers with the flag off and checks that every entry comes back 0 and that
the main outputs are bit-identical to a call with the flag on, over the
kernels that write them: the split decode path (combine kernel), unsplit
rows, the D = 128 kernel, and the indexer's one-row, four-row, fused and
general top-k paths.
"""
import numpy as np
import pytest
import torch

INT64_MAX = 9223372036854775807

pytestmark = pytest.mark.gpu


def _lib():
    from dsa_triton_ascend_amd import _lib as L
    return L, L.load()


@pytest.mark.parametrize("B,S1,N1,D,K,mode", [
    (2, 1, 128, 512, 2048, 0),     # decode: token splits, statistics from the combine kernel
    (1, 512, 128, 512, 256, 3),    # rows without splits (causal)
    (2, 64, 64, 128, 512, 3),      # the D = 128 kernel
    (3, 1, 16, 256, 1024, 0),      # D = 256, 16 heads
])
def test_sfa_statistics_zero_when_not_requested(B, S1, N1, D, K, mode):
    L, lib = _lib()
    g = torch.Generator(device="cuda").manual_seed(B * 1000 + S1 + N1 + D)
    bf = torch.bfloat16
    S2 = max(K, S1) * 2
    q = torch.randn(B, S1, N1, D, generator=g, device="cuda").to(bf)
    qr = torch.randn(B, S1, N1, 64, generator=g, device="cuda").to(bf)
    k = torch.randn(B, S2, 1, D, generator=g, device="cuda").to(bf)
    kr = torch.randn(B, S2, 1, 64, generator=g, device="cuda").to(bf)
    si = torch.stack([torch.randperm(S2, generator=g, device="cuda")[:K] for _ in range(B * S1)])
    si[0, K // 2:] = -1
    si = si.to(torch.int32).reshape(B, S1, 1, K).contiguous()
    rows = B * S1
    stream = L.stream_handle(torch.device("cuda:0"))
    ws_bytes = lib.dsa_sfa_fwd_workspace_size(rows, N1, D, K, 1)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    print(f"[unrequested] sfa B={B} S1={S1} N1={N1} D={D} K={K} mode={mode} ws={ws_bytes}", flush=True)

    def call(ret):
        out = torch.full((B, S1, N1, D), float("nan"), dtype=bf, device="cuda")
        smax = torch.full((B, 1, S1, N1), float("nan"), device="cuda")
        ssum = torch.full((B, 1, S1, N1), float("nan"), device="cuda")
        st = lib.dsa_sfa_fwd(q.data_ptr(), qr.data_ptr(), k.data_ptr(), kr.data_ptr(), si.data_ptr(),
                             out.data_ptr(), smax.data_ptr(), ssum.data_ptr(), None, None, None,
                             B, S1, S2, N1, D, 64, K, rows, B * S2, 0, 0, 1, mode, INT64_MAX, INT64_MAX,
                             L.LAYOUT["BSND"], L.LAYOUT["BSND"], L.DTYPE_BF16, 1.0 / np.sqrt(D + 64), ret,
                             ws.data_ptr(), ws_bytes, stream)
        L.check(st, "dsa_sfa_fwd")
        torch.cuda.synchronize()
        return out.cpu(), smax.cpu(), ssum.cpu()

    o1, m1, s1 = call(1)
    o0, m0, s0 = call(0)
    assert torch.isfinite(m1).all() and torch.isfinite(s1).all() and (s1 > 0).any()
    assert torch.equal(o0.view(torch.int16), o1.view(torch.int16)), "output differs with the statistics off"
    assert (m0 == 0).all() and (s0 == 0).all(), "statistics not zeroed when not requested"
    assert not torch.signbit(m0).any() and not torch.signbit(s0).any()


def test_sfa_api_statistics_zero_over_reused_memory():
    """The Python API allocates the statistics without a fill: poison the
    allocator's cached blocks of that size first."""
    import dsa_triton_ascend_amd as dsa
    g = torch.Generator(device="cuda").manual_seed(5)
    bf = torch.bfloat16
    B, N1, D, K, S2 = 4, 128, 512, 1024, 4096
    q = torch.randn(B, 1, N1, D, generator=g, device="cuda").to(bf)
    qr = torch.randn(B, 1, N1, 64, generator=g, device="cuda").to(bf)
    k = torch.randn(B, S2, 1, D, generator=g, device="cuda").to(bf)
    kr = torch.randn(B, S2, 1, 64, generator=g, device="cuda").to(bf)
    si = torch.stack([torch.randperm(S2, generator=g, device="cuda")[:K] for _ in range(B)])
    si = si.to(torch.int32).reshape(B, 1, 1, K).contiguous()
    for _ in range(3):
        junk = [torch.full((B, 1, 1, N1), float("nan"), device="cuda") for _ in range(8)]
        del junk
        out, smax, ssum = dsa.sparse_flash_attention_triton(q, k, k, si, scale_value=0.05, query_rope=qr,
                                                            key_rope=kr)
        torch.cuda.synchronize()
        assert (smax == 0).all() and (ssum == 0).all()
        assert torch.isfinite(out.float()).all()


def _li_call(lib, L, q, k, w, values, ret, B, S1, S2, N1, K, mode):
    rows = B * S1
    idx = torch.empty(B, S1, 1, K, dtype=torch.int32, device="cuda")
    ws_bytes = lib.dsa_li_fwd_workspace_size(rows, 1, S2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    st = lib.dsa_li_fwd(q.data_ptr(), k.data_ptr(), w.data_ptr(), None, None, idx.data_ptr(), values.data_ptr(),
                        B, S1, S2, N1, 1, 128, K, rows, B * S2, mode, L.LAYOUT["BSND"], L.LAYOUT["BSND"],
                        L.DTYPE_BF16, L.DTYPE_FP32, ret, ws.data_ptr(), ws_bytes,
                        L.stream_handle(torch.device("cuda:0")))
    L.check(st, "dsa_li_fwd")
    torch.cuda.synchronize()
    return idx.cpu()


@pytest.mark.parametrize("B,S1,S2,N1,K,mode,kind", [
    (4, 1, 32768, 64, 2048, 0, "random"),   # one-row top-k (decode)
    (1, 2048, 2048, 64, 512, 3, "random"),  # scores and top-k in one launch (four rows per workgroup)
    (2, 700, 6000, 32, 1024, 3, "random"),  # four-row top-k kernel after the score kernel
    (2, 3, 9000, 64, 2048, 0, "zero"),      # all-equal scores: the general selection
])
def test_indexer_values_zero_when_not_requested(B, S1, S2, N1, K, mode, kind):
    L, lib = _lib()
    g = torch.Generator(device="cuda").manual_seed(S1 + S2 + K)
    bf = torch.bfloat16
    q = torch.randn(B, S1, N1, 128, generator=g, device="cuda").to(bf)
    k = torch.randn(B, S2, 1, 128, generator=g, device="cuda").to(bf)
    w = torch.rand(B, S1, N1, generator=g, device="cuda")
    if kind == "zero":
        w.zero_()
    print(f"[unrequested] indexer B={B} S1={S1} S2={S2} N1={N1} K={K} mode={mode} {kind}", flush=True)
    v1 = torch.full((B, S1, 1, K), float("nan"), dtype=bf, device="cuda")
    i1 = _li_call(lib, L, q, k, w, v1, 1, B, S1, S2, N1, K, mode)
    v0 = torch.full((B, S1, 1, K), float("nan"), dtype=bf, device="cuda")
    i0 = _li_call(lib, L, q, k, w, v0, 0, B, S1, S2, N1, K, mode)
    assert torch.equal(i0, i1), "indices differ with the values off"
    v1c = v1.float().cpu()
    assert not torch.isnan(v1c).any(), "requested values left unwritten"
    assert (v0.float().cpu() == 0).all(), "values not zeroed when not requested"


def test_indexer_api_values_zero_over_reused_memory():
    """The Python API allocates the values without a fill (BSND and paged
    keys): poison the allocator's cached blocks of that size first."""
    import dsa_triton_ascend_amd as dsa
    g = torch.Generator(device="cuda").manual_seed(9)
    bf = torch.bfloat16
    B, S2, N1, K, page = 4, 8192, 64, 2048, 64
    q = torch.randn(B, 1, N1, 128, generator=g, device="cuda").to(bf)
    k = torch.randn(B, S2, 1, 128, generator=g, device="cuda").to(bf)
    w = torch.rand(B, 1, N1, generator=g, device="cuda")
    bt = torch.arange(B * S2 // page, device="cuda", dtype=torch.int32).reshape(B, S2 // page)
    kc = k.reshape(B * S2 // page, page, 1, 128)
    for paged in (False, True):
        for _ in range(2):
            junk = [torch.full((B, 1, 1, K), float("nan"), dtype=bf, device="cuda") for _ in range(8)]
            del junk
            if paged:
                idx, val = dsa.lightning_indexer_triton(q, kc, w, actual_seq_lengths_key=[S2] * B, block_table=bt,
                                                        layout_key="PA_BSND", sparse_count=K, sparse_mode=0)
            else:
                idx, val = dsa.lightning_indexer_triton(q, k, w, sparse_count=K, sparse_mode=0)
            torch.cuda.synchronize()
            assert (val.float() == 0).all(), f"values not zero (paged={paged})"
            assert ((idx >= 0) & (idx < S2)).all()
