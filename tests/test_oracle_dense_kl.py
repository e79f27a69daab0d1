"""Pins for the dense indexer LSE / dense KL-loss oracle (CPU only).

The reference's dense test compares against CANN on an NPU and a NumPy LSE
written in the test itself (test_dense_loss_backward_triton.py:101-138); it
holds no vectors.  The restatement is pinned by: an independent scalar
brute force of the LSE; the logsumexp identity; the sparse KL oracle (itself
pinned by the reference goldens) on the same problem with every visible key
selected, which the dense KL must equal up to where the 1e-8 guard sits;
finite differences of the loss with the index statistics recomputed from the
perturbed inputs (the setting in which dI = softmax(I) - p is the exact
gradient); and GQA reducing to MQA when the key heads are copies.
"""
import math

import numpy as np

from oracle.dense_kl import dense_index_lse, dense_kl_bwd
from oracle.kl import kl_loss_bwd


def _problem(rng, B=1, S1=3, S2=7, N1=4, N2=1, D=8, Dr=4, Ni=3, Di=8, rope=True):
    q = rng.randn(B, S1, N1, D) * 0.5
    k = rng.randn(B, S2, N2, D) * 0.5
    qr = rng.randn(B, S1, N1, Dr) * 0.5 if rope else None
    kr = rng.randn(B, S2, N2, Dr) * 0.5 if rope else None
    qi = rng.randn(B, S1, Ni, Di)
    ki = rng.randn(B, S2, 1, Di)
    w = np.abs(rng.randn(B, S1, Ni))
    scale = 1 / math.sqrt(D + (Dr if rope else 0))
    return q, k, qr, kr, qi, ki, w, scale


def _teacher_stats(q, k, qr, kr, scale, aq=None, ak=None):
    """Exact causal softmax stats [B, N2, S1, G] over the visible keys."""
    B, S1, N1, _ = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    aq = [S1] * B if aq is None else aq
    ak = [S2] * B if ak is None else ak
    smax = np.zeros((B, N2, S1, G)); ssum = np.zeros((B, N2, S1, G))
    for b in range(B):
        for s1 in range(min(S1, aq[b])):
            L = min(max(ak[b] - aq[b] + s1 + 1, 0), S2)
            if L <= 0:
                continue
            for h in range(N1):
                n2, g = h // G, h % G
                s = q[b, s1, h] @ k[b, :L, n2].T
                if qr is not None:
                    s = s + qr[b, s1, h] @ kr[b, :L, n2].T
                s = s * scale
                smax[b, n2, s1, g] = s.max()
                ssum[b, n2, s1, g] = np.exp(s - s.max()).sum()
    return smax, ssum


def test_dense_lse_matches_scalar_brute_force():
    rng = np.random.RandomState(1)
    _, _, _, _, qi, ki, w, _ = _problem(rng, B=2, S1=4, S2=6)
    aq, ak = [4, 3], [6, 2]
    m, s = dense_index_lse(qi, ki, w, aq, ak)
    for b in range(2):
        for s1 in range(4):
            vis = [t for t in range(6) if s1 < aq[b] and t < min(max(ak[b] - aq[b] + s1 + 1, 0), 6)]
            if not vis:
                assert m[b, 0, s1] == -np.inf and s[b, 0, s1] == 0
                continue
            I = []
            for t in vis:
                tot = 0.0
                for g in range(qi.shape[2]):
                    dot = sum(float(qi[b, s1, g, d]) * float(ki[b, t, 0, d]) for d in range(qi.shape[3]))
                    tot += float(w[b, s1, g]) * max(dot, 0.0)
                I.append(tot)
            mm = max(I)
            assert abs(m[b, 0, s1] - mm) < 1e-12
            assert abs(s[b, 0, s1] - sum(math.exp(x - mm) for x in I)) < 1e-12
            # logsumexp identity
            assert abs(mm + math.log(s[b, 0, s1]) - math.log(sum(math.exp(x) for x in I))) < 1e-9


def test_dense_kl_equals_sparse_kl_with_all_visible_keys():
    """MQA: the dense backward is the sparse one with sparse_indices = 0..S2-1
    (every visible key selected, kernel line 107 takes the visible prefix);
    they differ only in where the 1e-8 guard of the student sits."""
    rng = np.random.RandomState(2)
    B, S1, S2 = 2, 4, 9
    q, k, qr, kr, qi, ki, w, scale = _problem(rng, B=B, S1=S1, S2=S2, N1=4, N2=1)
    aq, ak = [4, 3], [9, 7]
    smax, ssum = _teacher_stats(q, k, qr, kr, scale, aq, ak)
    d = dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale, act_q=aq, act_k=ak)
    si = np.tile(np.arange(S2, dtype=np.int32), (B, S1, 1, 1))
    sp = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, aq, ak,
                     compute_dtype=np.float64)
    for key in ("dQueryIndex", "dKeyIndex", "dW", "loss"):
        np.testing.assert_allclose(d[key], sp[key], rtol=1e-6, atol=1e-9, err_msg=key)


def test_dense_kl_gradients_match_finite_differences():
    """With the index statistics recomputed from the inputs and p summing to
    one, dI = softmax(I) - p is the gradient of the loss in I."""
    rng = np.random.RandomState(3)
    q, k, qr, kr, qi, ki, w, scale = _problem(rng, S1=3, S2=6, N1=4, N2=2)
    smax, ssum = _teacher_stats(q, k, qr, kr, scale)
    r = dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale)
    np.testing.assert_allclose(r["p"].sum(-1), 1.0, rtol=1e-6)

    def loss(qi_, ki_, w_):
        return float(dense_kl_bwd(q, k, qr, kr, qi_, ki_, w_, smax, ssum, scale)["loss"][0])

    eps = 1e-6
    for which, arr, g in (("qi", qi, r["dQueryIndex"]), ("ki", ki, r["dKeyIndex"]), ("w", w, r["dW"])):
        for idx in list(np.ndindex(arr.shape))[::max(1, arr.size // 15)]:
            args = {"qi": qi, "ki": ki, "w": w}
            a = arr.copy(); a[idx] += eps; args[which] = a
            lp = loss(args["qi"], args["ki"], args["w"])
            a = arr.copy(); a[idx] -= eps; args[which] = a
            lm = loss(args["qi"], args["ki"], args["w"])
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - g[idx]) < 1e-5 * max(1.0, abs(fd)), (which, idx, fd, g[idx])


def test_dense_kl_gqa_with_copied_key_heads_is_mqa():
    rng = np.random.RandomState(4)
    q, k, qr, kr, qi, ki, w, scale = _problem(rng, S1=3, S2=5, N1=4, N2=1)
    k2, kr2 = np.repeat(k, 2, axis=2), np.repeat(kr, 2, axis=2)
    sm1, ss1 = _teacher_stats(q, k, qr, kr, scale)
    sm2, ss2 = _teacher_stats(q, k2, qr, kr2, scale)
    a = dense_kl_bwd(q, k, qr, kr, qi, ki, w, sm1, ss1, scale)
    b = dense_kl_bwd(q, k2, qr, kr2, qi, ki, w, sm2, ss2, scale)
    for key in ("dQueryIndex", "dKeyIndex", "dW", "loss"):
        np.testing.assert_allclose(a[key], b[key], rtol=1e-12, atol=1e-14, err_msg=key)


def test_dense_kl_given_stats_are_used_and_invalid_rows_are_zero():
    """The backward takes the index statistics as given (the reference's
    with-index core): scaling isum by c scales the student by 1/c.  A row
    with isum = 0 (has_valid false) contributes nothing."""
    rng = np.random.RandomState(5)
    q, k, qr, kr, qi, ki, w, scale = _problem(rng, S1=3, S2=6)
    smax, ssum = _teacher_stats(q, k, qr, kr, scale)
    m, s = dense_index_lse(qi, ki, w)
    r1 = dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale, m.reshape(-1), s.reshape(-1))
    s2 = s.reshape(-1).copy(); s2[1] *= 2.0; s2[2] = 0.0
    r2 = dense_kl_bwd(q, k, qr, kr, qi, ki, w, smax, ssum, scale, m.reshape(-1), s2)
    np.testing.assert_allclose(r2["student"][0, 1], r1["student"][0, 1] / 2, rtol=1e-12)
    assert np.all(r2["dI"][0, 2] == 0) and np.all(r2["dQueryIndex"][0, 2] == 0) and np.all(r2["dW"][0, 2] == 0)
    np.testing.assert_array_equal(r2["student"][0, 0], r1["student"][0, 0])
