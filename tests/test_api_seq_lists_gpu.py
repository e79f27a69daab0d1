"""Sequence-length lists through the Python APIs.

The APIs keep the device copy of a plain-list length argument in a cache
keyed by the list's contents (a pageable host-to-device copy per call would
wait for the stream's queued kernels).  These tests check that a list gives
the same outputs as the equivalent tensor, that a list mutated in place
between calls is seen with its new contents, and that results stay right
after more distinct lists than the cache holds.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _decode_inputs(B, ctx, page, K, seed=11):
    g = torch.Generator(device="cuda").manual_seed(seed)
    bf = torch.bfloat16
    nblk = B * ctx // page
    t = dict(cache=torch.randn(nblk, page, 1, 512, generator=g, device="cuda").to(bf),
             cache_r=torch.randn(nblk, page, 1, 64, generator=g, device="cuda").to(bf),
             q=torch.randn(B, 1, 128, 512, generator=g, device="cuda").to(bf),
             qr=torch.randn(B, 1, 128, 64, generator=g, device="cuda").to(bf),
             bt=torch.randperm(nblk, generator=g, device="cuda").to(torch.int32).reshape(B, ctx // page))
    si = torch.stack([torch.randperm(ctx, generator=g, device="cuda")[:K] for _ in range(B)])
    t["si"] = si.to(torch.int32).reshape(B, 1, 1, K).contiguous()
    return t


def _sfa(t, lens):
    import dsa_triton_ascend_amd as dsa
    out, smax, ssum = dsa.sparse_flash_attention_triton(
        t["q"], t["cache"], t["cache"], t["si"], scale_value=1 / math.sqrt(576), block_table=t["bt"],
        actual_seq_lengths_kv=lens, query_rope=t["qr"], key_rope=t["cache_r"], layout_kv="PA_BSND",
        return_softmax_lse=True)
    torch.cuda.synchronize()
    return out, smax, ssum


def _same(a, b):
    return all(torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y) for x, y in zip(a, b))


def test_sfa_length_list_matches_tensor_and_follows_mutation():
    B, ctx, page, K = 3, 4096, 64, 1024
    t = _decode_inputs(B, ctx, page, K)
    lens = [ctx, ctx // 2, 700]
    r_list = _sfa(t, lens)
    r_tens = _sfa(t, torch.tensor(lens, dtype=torch.int32, device="cuda"))
    assert _same(r_list, r_tens)
    # the same list object with new contents
    lens[1] = 1500
    lens[2] = ctx
    r_list2 = _sfa(t, lens)
    r_tens2 = _sfa(t, torch.tensor(lens, dtype=torch.int32, device="cuda"))
    assert _same(r_list2, r_tens2)
    assert not _same(r_list, r_list2), "new lengths must change the outputs"


def test_sfa_length_lists_beyond_cache_capacity():
    import importlib
    # the module (the package re-exports a function of the same name)
    sfa_mod = importlib.import_module("dsa_triton_ascend_amd.sparse_flash_attention")
    B, ctx, page, K = 2, 2048, 64, 512
    t = _decode_inputs(B, ctx, page, K, seed=12)
    first = [ctx, 999]
    ref = _sfa(t, torch.tensor(first, dtype=torch.int32, device="cuda"))
    assert _same(_sfa(t, first), ref)
    for i in range(sfa_mod._SEQ_CACHE_MAX + 6):
        _sfa(t, [ctx - i, 1000 + i])
    assert len(sfa_mod._SEQ_CACHE) <= sfa_mod._SEQ_CACHE_MAX
    assert _same(_sfa(t, first), ref)


def test_indexer_length_list_matches_tensor():
    import dsa_triton_ascend_amd as dsa
    g = torch.Generator(device="cuda").manual_seed(13)
    bf = torch.bfloat16
    B, S1, S2, N1, K = 2, 4, 3000, 64, 512
    q = torch.randn(B, S1, N1, 128, generator=g, device="cuda").to(bf)
    k = torch.randn(B, S2, 1, 128, generator=g, device="cuda").to(bf)
    w = torch.rand(B, S1, N1, generator=g, device="cuda")
    lq, lk = [S1, 3], [S2, 2100]
    a = dsa.lightning_indexer_triton(q, k, w, actual_seq_lengths_query=lq, actual_seq_lengths_key=lk,
                                     sparse_count=K, sparse_mode=3, return_value=True)
    b = dsa.lightning_indexer_triton(q, k, w, actual_seq_lengths_query=torch.tensor(lq, device="cuda"),
                                     actual_seq_lengths_key=torch.tensor(lk, device="cuda"),
                                     sparse_count=K, sparse_mode=3, return_value=True)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1].view(torch.int16), b[1].view(torch.int16))
