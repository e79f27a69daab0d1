"""GPU tests of the autograd pairing (``dsa_triton_ascend_amd.autograd``).

The reference's bprop recipe for MLA-absorb returns ``dk + dv`` for the
shared key (sparse_flash_attention_grad_triton.py:30-71). The checks here:

* the gradients that ``loss.backward()`` produces through
  ``sparse_flash_attention_train`` against a float64 torch-autograd
  reference on the CPU. That reference is independent of the kernel
  derivation: it gathers the selected rows with the kernel's per-entry masks
  and differentiates plain softmax attention whose value is ``key[..., :D]``.
  Tolerances are those of the direct backward tests: rtol 2e-2 / atol 2e-3,
  with atol scaled by the largest entry for dK, which sums many rows;
* the same gradients against the direct ``sparse_flash_attention_grad_triton``
  outputs (``dk + dv``);
* the indexer KL loss as a differentiable scalar: the gradients of
  ``(c * loss).backward()`` against a float64 torch-autograd reference of
  KL(p || softmax(I)), with the teacher p taken from statistics over the same
  selected set (p then sums to 1, and autograd's dI equals the kernel's
  softmax(I) - p), and against c times the direct outputs.
"""
import numpy as np
import pytest
import torch

from tests.helpers import dev, sfa_inputs, sparse_indices, to_dtype_np

pytestmark = pytest.mark.gpu


def _api():
    import dsa_triton_ascend_amd as dsa
    return dsa


def _sfa_torch_ref(q, k, qr, kr, si, scale, mode):
    """float64 CPU autograd reference of the BSND forward (kernel masks)."""
    B, S1, N1, D = q.shape
    S2 = k.shape[1]
    rows = []
    for b in range(B):
        for s1 in range(S1):
            thr = S2 if mode == 0 else S2 - S1 + s1 + 1
            ids = [int(t) for t in si[b, s1, 0] if 0 <= t < thr and t < S2]
            if not ids:
                rows.append(torch.zeros(N1, D, dtype=torch.float64))
                continue
            ix = torch.tensor(ids)
            kf = torch.cat([k[b, ix, 0], kr[b, ix, 0]], dim=-1)          # [n, D+64]
            qf = torch.cat([q[b, s1], qr[b, s1]], dim=-1)                # [N1, D+64]
            p = torch.softmax((qf @ kf.T) * scale, dim=-1)
            rows.append(p @ k[b, ix, 0])
    return torch.stack(rows).reshape(B, S1, N1, D)


def _close(got, exp, rtol, atol, what):
    g = got.detach().float().cpu().double()
    err = (g - exp).abs()
    tol = atol + rtol * exp.abs()
    bad = err > tol
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} out of tolerance, max err {float(err.max()):.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("mode", [0, 3])
def test_sfa_train_grads_match_torch_reference(dtype, mode):
    print(f"[autograd sfa] mode={mode} {dtype}", flush=True)
    dsa = _api()
    B, S1, S2, N1, D, K = 1, 8, 64, 16, 128, 32
    q, k, qr, kr = sfa_inputs(B, S1, S2, N1, D, dtype, seed=11)
    si = sparse_indices(B, S1, S2, K, 1, mode, seed=13)
    scale = 1.0 / np.sqrt(D + 64)
    g = np.random.RandomState(5).randn(B, S1, N1, D).astype(np.float32)

    ref_in = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, qr, kr)]
    out_ref = _sfa_torch_ref(*ref_in, si, scale, mode)
    (out_ref * torch.tensor(g)).sum().backward()
    dq_r, dk_r, dqr_r, dkr_r = (t.grad for t in ref_in)

    gq, gk, gqr, gkr = (dev(x, dtype).requires_grad_(True) for x in (q, k, qr, kr))
    out, smax, ssum = dsa.sparse_flash_attention_train(
        gq, gk, dev(si, torch.int32), scale_value=scale, query_rope=gqr, key_rope=gkr,
        sparse_mode=mode)
    (out.float() * dev(g, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    _close(out, out_ref.detach(), 2e-2, 2e-3, "attention_out")
    _close(gq.grad, dq_r, 2e-2, 2e-3, "d_query")
    _close(gqr.grad, dqr_r, 2e-2, 2e-3, "d_query_rope")
    _close(gk.grad, dk_r, 2e-2, 2e-3 * float(dk_r.abs().max()), "d_key (dk + dv)")
    _close(gkr.grad, dkr_r, 2e-2, 2e-3 * float(dkr_r.abs().max()), "d_key_rope")

    # the same gradients from the direct backward API
    dq, dk, dv, dqr, dkr = dsa.sparse_flash_attention_grad_triton(
        gq.detach(), gk.detach(), gk.detach(), dev(si, torch.int32), dev(g, dtype), out.detach(),
        smax, ssum, scale_value=scale, query_rope=gqr.detach(), key_rope=gkr.detach(), sparse_mode=mode)
    torch.cuda.synchronize()
    # dq / dq_rope are per-row sums (deterministic); dk / dk_rope / dv come
    # from fp32 atomics, whose order differs between the two calls
    assert torch.equal(gq.grad, dq) and torch.equal(gqr.grad, dqr)
    # the merged gradient is rounded once; dk and dv were each rounded, so
    # their sum may differ by half an ulp of each plus one of the result
    # (x 2 for the atomic order), relative to the dtype's mantissa
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    dkv = dk.float() + dv.float()
    bound = 2 * eps * (dk.float().abs() + dv.float().abs() + dkv.abs()) + 1e-3 * float(dkv.abs().max())
    assert bool(((gk.grad.float() - dkv).abs() <= bound).all()), "merged d_key vs dk + dv"
    _close(gk.grad, dk_r, 2e-2, 2e-3 * float(dk_r.abs().max()), "merged d_key vs reference")
    torch.testing.assert_close(gkr.grad.float(), dkr.float(), rtol=1e-2, atol=1e-3 * float(dkr.float().abs().max()))


def test_sfa_train_tnd_and_module():
    print("[autograd sfa] TND and module", flush=True)
    dsa = _api()
    dtype = torch.bfloat16
    B, S, N1, D, K = 2, 24, 8, 128, 16
    q, k, qr, kr = sfa_inputs(B, S, S, N1, D, dtype, seed=21)
    si = sparse_indices(B, S, S, K, 1, 3, seed=23)
    scale = 1.0 / np.sqrt(D + 64)
    g = np.random.RandomState(7).randn(B, S, N1, D).astype(np.float32)
    cu = [S, 2 * S]

    def run(layout):
        ins = [dev(x, dtype).requires_grad_(True) for x in (q, k, qr, kr)]
        if layout == "TND":
            qq, kk, qqr, kkr = (t.reshape(B * S, *t.shape[2:]) for t in ins)
            sii = dev(si.reshape(B * S, 1, K), torch.int32)
            out, _, _ = dsa.sparse_flash_attention_train(
                qq, kk, sii, scale_value=scale, query_rope=qqr, key_rope=kkr, actual_seq_lengths_query=cu,
                actual_seq_lengths_kv=cu, layout="TND", sparse_mode=3)
            out = out.reshape(B, S, N1, D)
        else:
            mod = dsa.SparseFlashAttentionTriton(scale_value=scale, sparse_mode=3)
            out, smax, ssum = mod(ins[0], ins[1], None, dev(si, torch.int32), ins[2], ins[3])
            assert float(smax.abs().sum()) == 0.0 and float(ssum.abs().sum()) == 0.0  # not requested
        (out.float() * dev(g, torch.float32)).sum().backward()
        torch.cuda.synchronize()
        return [t.grad.float().cpu() for t in ins]

    tnd, bsnd = run("TND"), run("BSND")
    for a, b, nm in zip(tnd, bsnd, ("dq", "dk", "dqr", "dkr")):
        # TND rows are BSND rows with a per-sequence base; the dK/dV atomic
        # order differs, so allow fp32 reassociation before the cast
        torch.testing.assert_close(a, b, rtol=1e-2, atol=1e-2 * float(b.abs().max()), msg=nm)


def _kl_inputs(dtype):
    rng = np.random.RandomState(31)
    B, S, N1, D, NI, DI, K = 1, 32, 16, 128, 8, 128, 16

    def t(shape):
        return to_dtype_np(rng.randn(*shape).astype(np.float16).astype(np.float32), dtype)

    q, k, qr, kr = t((B, S, N1, D)), t((B, S, 1, D)), t((B, S, N1, 64)), t((B, S, 1, 64))
    qi, ki = t((B, S, NI, DI)), t((B, S, 1, DI))
    w = rng.rand(B, S, NI).astype(np.float32)
    si = np.zeros((B, S, 1, K), np.int32)
    for s1 in range(S):
        n = min(K, s1 + 1)
        si[0, s1, 0, :n] = rng.choice(s1 + 1, size=n, replace=False)
    scale = 1.0 / np.sqrt(D + 64)
    # statistics over the same selected set: the teacher p sums to 1
    smax = np.zeros((B, 1, S, N1), np.float32)
    ssum = np.zeros((B, 1, S, N1), np.float32)
    for s1 in range(S):
        n = min(K, s1 + 1)
        ix = si[0, s1, 0, :n]
        sc = (q[0, s1].astype(np.float64) @ k[0, ix, 0].T + qr[0, s1].astype(np.float64) @ kr[0, ix, 0].T) * scale
        m = sc.max(axis=1)
        smax[0, 0, s1] = m
        ssum[0, 0, s1] = np.exp(sc - m[:, None]).sum(axis=1)
    return q, k, qr, kr, qi, ki, w, si, smax, ssum, scale


def _kl_torch_ref(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, clamped=False):
    """float64 CPU autograd of sum_rows KL(p || softmax(I)) over the first
    n = min(K, s1 + 1) slots (full lengths, sparse_mode 3)."""
    S, N1 = q.shape[1], q.shape[2]
    K = si.shape[3]
    total = torch.zeros((), dtype=torch.float64)
    for s1 in range(S):
        n = min(K, s1 + 1)
        ix = torch.tensor(si[0, s1, 0, :n].astype(np.int64))
        sc = (torch.tensor(q[0, s1], dtype=torch.float64) @ torch.tensor(k[0, :, 0], dtype=torch.float64)[ix].T
              + torch.tensor(qr[0, s1], dtype=torch.float64) @ torch.tensor(kr[0, :, 0], dtype=torch.float64)[ix].T) * scale
        pr = torch.exp(sc - torch.tensor(smax[0, 0, s1], dtype=torch.float64)[:, None]) \
            / torch.tensor(ssum[0, 0, s1], dtype=torch.float64)[:, None]
        p = pr.sum(0) / N1
        relu = torch.relu(qi[0, s1] @ ki[0, ix, 0].T)            # [NI, n]
        I = w[0, s1] @ relu
        if clamped:
            # the loss value: p and softmax(I) clamped at 1e-8 inside the log,
            # as the reference (sli_grad_kl_loss_numpy.py:111-117)
            pc = p.clamp_min(1e-8)
            total = total + (pc * (torch.log(pc) - torch.log(torch.softmax(I, dim=0).clamp_min(1e-8)))).sum()
        else:
            # the gradient: dI = softmax(I) - p is the derivative of the
            # unclamped KL (sli_grad_kl_loss_numpy.py:107-108)
            total = total + (p * (torch.log(p) - torch.log_softmax(I, dim=0))).sum()
    return total


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_kl_loss_autograd(dtype):
    print(f"[autograd kl] {dtype}", flush=True)
    dsa = _api()
    q, k, qr, kr, qi, ki, w, si, smax, ssum, scale = _kl_inputs(dtype)
    c = 3.0

    rqi, rki, rw = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (qi, ki, w))
    (c * _kl_torch_ref(q, k, qr, kr, rqi, rki, rw, si, smax, ssum, scale)).backward()
    with torch.no_grad():
        ref_loss = _kl_torch_ref(q, k, qr, kr, rqi, rki, rw, si, smax, ssum, scale, clamped=True)

    gqi, gki = dev(qi, dtype).requires_grad_(True), dev(ki, dtype).requires_grad_(True)
    gw = dev(w, torch.float32).requires_grad_(True)
    args = (dev(q, dtype), dev(k, dtype), dev(si, torch.int32), dev(smax, torch.float32),
            dev(ssum, torch.float32))
    loss = dsa.sparse_lightning_indexer_kl_loss(gqi, gki, gw, *args, query_rope=dev(qr, dtype),
                                                key_rope=dev(kr, dtype), scale_value=scale)
    (c * loss).sum().backward()
    torch.cuda.synchronize()
    assert abs(float(loss.detach()) - float(ref_loss)) <= 1e-3 * abs(float(ref_loss)) + 1e-4
    _close(gw.grad, rw.grad, 1e-3, 1e-5 * c, "d_weights")
    _close(gqi.grad, rqi.grad, 1e-2, 1e-3 * float(rqi.grad.abs().max()), "d_query_index")
    _close(gki.grad, rki.grad, 1e-2, 1e-3 * float(rki.grad.abs().max()), "d_key_index")

    # c times the direct operator's outputs
    d_qi, d_ki, d_w, loss2 = dsa.sparse_lightning_indexer_grad_kl_loss_triton(
        args[0], args[1], gqi.detach(), gki.detach(), gw.detach(), args[2], args[3], args[4],
        query_rope=dev(qr, dtype), key_rope=dev(kr, dtype), scale_value=scale)
    torch.cuda.synchronize()
    assert torch.equal(gqi.grad, (d_qi.float() * c).to(dtype))
    assert torch.equal(gki.grad, (d_ki.float() * c).to(dtype))
    assert torch.equal(gw.grad, d_w * c)
    assert torch.equal(loss, loss2)
