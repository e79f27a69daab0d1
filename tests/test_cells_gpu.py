"""GPU parity of the module (Cell) forms against the oracle.

Each module is built with the reference Cell's positional constructor order
and called with its ``construct`` argument order:

* ``SparseFlashAttentionTriton`` (sparse_flash_attention_triton.py:644-695),
  inference path (no input requires grad), BSND and PA_BSND;
* ``SparseFlashAttentionGradTriton`` (sparse_flash_attention_grad_triton.py:
  544-586);
* ``LightningIndexerTriton`` (lightning_indexer_triton.py:416-459), with
  ``return_value`` as its fifth positional argument;
* ``SparseLightningIndexerGradKLLossTriton``
  (sparse_lightning_indexer_grad_kl_loss_triton.py:467-515).

Tolerances as the functional suites: north star rtol 2e-2 / atol 2e-3 for SFA
outputs and per-row gradients (atol scaled by the largest magnitude for the
scatter-added key gradients), bit-exact top-k up to reassociation tie flips,
KL at rtol 1e-3 (dW, loss) / 1e-2 (dQi, dKi).
"""
import numpy as np
import pytest
import torch

from oracle.common import pa_to_bsnd
from oracle.indexer import indexer_scores
from oracle.kl import kl_loss_bwd
from oracle.sfa import sfa_fwd_bsnd
from oracle.sfa_grad import sfa_bwd_bsnd
from tests.helpers import assert_close, dev, sfa_inputs, sparse_indices, to_dtype_np

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def test_sfa_cell_inference_bsnd():
    import dsa_triton_ascend_amd as dsa
    print("[cell] SparseFlashAttentionTriton BSND", flush=True)
    B, S1, S2, N1, D, K = 2, 6, 200, 16, 512, 64
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=11)
    si = sparse_indices(B, S1, S2, K, 1, 3, seed=12)
    scale = 1.0 / np.sqrt(D + 64)
    # (scale_value, sparse_block_size, layout_query, layout_kv, sparse_mode, attention_mode, return_softmax_lse)
    cell = dsa.SparseFlashAttentionTriton(scale, 1, "BSND", "BSND", 3, 2, True)
    with torch.no_grad():
        out, smax, ssum = cell(dev(q, BF), dev(k, BF), dev(k, BF), dev(si, torch.int32), dev(qr, BF), dev(kr, BF))
    torch.cuda.synchronize()
    ref = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [S1] * B, [S2] * B, 1, 3, True, "float32", positions="kernel")
    assert_close(out.float().cpu().numpy(), ref[0], 2e-2, 2e-3, "out")
    assert_close(smax.cpu().numpy(), ref[1], 2e-2, 2e-3, "softmax_max")
    assert_close(ssum.cpu().numpy(), ref[2], 2e-2, 2e-3, "softmax_sum")
    # return_softmax_lse=False: the statistics are zeros (sparse_flash_attention_triton.py:527)
    cell = dsa.SparseFlashAttentionTriton(scale, 1, "BSND", "BSND", 3)
    out2, smax2, ssum2 = cell.construct(dev(q, BF), dev(k, BF), None, dev(si, torch.int32), dev(qr, BF),
                                        dev(kr, BF))
    assert torch.equal(out2, out) and not smax2.any() and not ssum2.any()


def test_sfa_cell_inference_paged():
    import dsa_triton_ascend_amd as dsa
    print("[cell] SparseFlashAttentionTriton PA_BSND", flush=True)
    B, N1, D, K, page, max_blocks = 3, 32, 512, 48, 16, 8
    S2 = page * max_blocks
    nblk = B * max_blocks + 2
    rng = np.random.RandomState(21)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float32), BF)  # noqa: E731
    q, qr = f(B, 1, N1, D), f(B, 1, N1, 64)
    cache, cache_r = f(nblk, page, 1, D), f(nblk, page, 1, 64)
    bt = rng.permutation(nblk)[:B * max_blocks].reshape(B, max_blocks).astype(np.int32)
    act_k = [S2, 70, 33]
    si = sparse_indices(B, 1, S2, K, 1, 0, act_q=[1] * B, act_k=act_k, seed=22)
    scale = 1.0 / np.sqrt(D + 64)
    cell = dsa.SparseFlashAttentionTriton(scale, 1, "BSND", "PA_BSND", 0, 2, True, block_size=page)
    out, smax, ssum = cell(dev(q, BF), dev(cache, BF), None, dev(si, torch.int32), dev(qr, BF), dev(cache_r, BF),
                           None, act_k, dev(bt, torch.int32))
    torch.cuda.synchronize()
    k = pa_to_bsnd(cache, bt, S2)
    kr = pa_to_bsnd(cache_r, bt, S2)
    ref = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [1] * B, act_k, 1, 0, True, "float32", positions="kernel")
    assert_close(out.float().cpu().numpy(), ref[0], 2e-2, 2e-3, "out")
    assert_close(smax.cpu().numpy(), ref[1], 2e-2, 2e-3, "softmax_max")
    assert_close(ssum.cpu().numpy(), ref[2], 2e-2, 2e-3, "softmax_sum")


def test_sfa_grad_cell():
    import dsa_triton_ascend_amd as dsa
    print("[cell] SparseFlashAttentionGradTriton", flush=True)
    B, S1, S2, N1, D, K = 1, 12, 256, 64, 512, 96
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, BF, seed=31)
    do = to_dtype_np(np.random.RandomState(32).randn(B, S1, N1, D).astype(np.float32), BF)
    si = sparse_indices(B, S1, S2, K, 1, 3, seed=33)
    scale = 1.0 / np.sqrt(D + 64)
    out, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [S1], [S2], 1, 3, True, "float32", positions="kernel")
    out = to_dtype_np(out, BF)
    # (scale_value, sparse_block_size, layout, sparse_mode)
    cell = dsa.SparseFlashAttentionGradTriton(scale, 1, "BSND", 3)
    got = cell(dev(q, BF), dev(k, BF), dev(k, BF), dev(si, torch.int32), dev(do, BF), dev(out, BF),
               dev(smax, torch.float32), dev(ssum, torch.float32), dev(qr, BF), dev(kr, BF))
    torch.cuda.synchronize()
    exp = sfa_bwd_bsnd(q, k, si, do, out, smax, ssum, qr, kr, scale, [S1], [S2], 1, 3, "float32",
                       positions="kernel", guard_sum=True)
    for name, g, e in zip(("dq", "dk", "dv", "dqr", "dkr"), got, exp):
        g = g.float().cpu().numpy()
        assert g.shape == e.shape, name
        atol = 2e-3 if name in ("dq", "dqr") else 2e-3 * max(1.0, float(np.abs(e).max()))
        assert_close(g, e, 2e-2, atol, name)


def test_lightning_indexer_cell_returns_values():
    import dsa_triton_ascend_amd as dsa
    from tests.test_li_gpu import _check_topk_with_ties, _inputs
    print("[cell] LightningIndexerTriton", flush=True)
    B, S1, S2, N1, D, k = 2, 5, 600, 64, 128, 128
    q, kk, w = _inputs(B, S1, S2, N1, 1, D, BF, seed=41)
    # (sparse_count, sparse_mode, layout_query, layout_key, return_value)
    cell = dsa.LightningIndexerTriton(k, 3, "BSND", "BSND", True)
    idx, val = cell(dev(q, BF), dev(kk, BF), dev(w, torch.float32))
    torch.cuda.synchronize()
    idx, val = idx.cpu().numpy(), val.float().cpu().numpy()
    sc = indexer_scores(q, kk, w, [S1] * B, [S2] * B, 3)
    for b in range(B):
        for s in range(S1):
            rs = sc[b, s]
            tol = np.full(1, 1e-5 * np.abs(np.where(np.isfinite(rs), rs, 0)).max() + 1e-4)
            _check_topk_with_ties(idx[b, s], rs, k, tol, f"row ({b},{s})")
            ii = idx[b, s, 0]
            exp_v = to_dtype_np(np.where(ii >= 0, rs[0, np.maximum(ii, 0)], -np.inf), BF)
            fin = ii >= 0
            assert np.all(np.abs(val[b, s, 0][fin] - exp_v[fin]) <= 1e-2 * np.abs(exp_v[fin]) + 1e-3)
            assert np.array_equal(np.isneginf(val[b, s, 0]), ~fin)
    assert np.abs(val[np.isfinite(val)]).max() > 0, "return_value=True must return the values"


def test_kl_loss_cell():
    import dsa_triton_ascend_amd as dsa
    print("[cell] SparseLightningIndexerGradKLLossTriton", flush=True)
    B, S1, S2, N1, D, Ni, topK = 1, 24, 24, 32, 512, 16, 16
    rng = np.random.RandomState(51)
    f = lambda *s: to_dtype_np(rng.randn(*s).astype(np.float32), BF)  # noqa: E731
    q, k, qr, kr = f(B, S1, N1, D), f(B, S2, 1, D), f(B, S1, N1, 64), f(B, S2, 1, 64)
    qi, ki = f(B, S1, Ni, 128), f(B, S2, 1, 128)
    w = rng.rand(B, S1, Ni).astype(np.float32)
    si = sparse_indices(B, S1, S2, topK, 1, 3, seed=52)
    si[si < 0] = 0
    scale = 1.0 / np.sqrt(D + 64)
    _, smax, ssum = sfa_fwd_bsnd(q, k, si, qr, kr, scale, [S1], [S2], 1, 3, True, "float32", positions="kernel")
    # (scale_value, layout, sparse_mode)
    cell = dsa.SparseLightningIndexerGradKLLossTriton(scale, "BSND", 3)
    dqi, dki, dw, loss = cell(dev(q, BF), dev(k, BF), dev(qi, BF), dev(ki, BF), dev(w, torch.float32),
                              dev(si, torch.int32), dev(smax, torch.float32), dev(ssum, torch.float32),
                              dev(qr, BF), dev(kr, BF))
    torch.cuda.synchronize()
    ref = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, compute_dtype=np.float64)
    assert dqi.dtype == BF and dki.dtype == BF and dw.dtype == torch.float32 and loss.shape == (1,)
    assert_close(dw.cpu().numpy(), ref["dW"], 1e-3, 1e-5, "dW")
    assert_close(loss.cpu().numpy(), ref["loss"], 1e-3, 1e-6, "loss")
    for name, g, e in (("dQi", dqi, ref["dQueryIndex"]), ("dKi", dki, ref["dKeyIndex"])):
        assert_close(g.float().cpu().numpy(), e, 1e-2, 1e-3 * float(np.abs(e).max()) + 1e-6, name)
