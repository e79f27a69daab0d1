"""Pins for the lightning-indexer and KL-loss oracles (CPU only).

Indexer: an independent scalar brute force of the score rule, basis-vector
keys with known scores, N1=1 / w=1 reducing to ReLU(q.k), tied scores coming
out in ascending index, the -1 count per row, and ``torch.sort(stable=True)``
as a second library ordering.  The reference holds no indexer vectors
(its only indexer test compares against CANN on an NPU, test_li_triton.py:83-128).

KL: the golden module cannot be imported here (it imports mindspore at module
level, sli_grad_kl_loss_numpy.py:6-8), so the restatement is pinned by
finite differences of the loss in fp64 when the teacher distribution sums
to one, by KL >= 0, by KL = 0 when softmax(I) equals the teacher, by
sum_k dI = 1 - sum_k p, and by an independent scalar brute force.
"""
import math

import numpy as np
import pytest

from oracle.indexer import indexer_scores, stable_topk, lightning_indexer, visible_limit
from oracle.kl import kl_loss_bwd


# ---------------------------------------------------------------------------
# indexer
# ---------------------------------------------------------------------------
def _brute_scores(q, k, w, aq, ak, mode):
    B, S1, N1, D = q.shape
    S2, N2 = k.shape[1], k.shape[2]
    G = N1 // N2
    out = np.full((B, S1, N2, S2), -np.inf)
    for b in range(B):
        for s1 in range(S1):
            for n2 in range(N2):
                for s2 in range(S2):
                    vis = s1 < aq[b] and s2 < ak[b]
                    if mode == 3:
                        vis = vis and s2 < min(max(ak[b] - aq[b] + s1 + 1, 0), S2)
                    if not vis:
                        continue
                    tot = 0.0
                    for g in range(G):
                        h = n2 * G + g
                        dot = sum(float(q[b, s1, h, d]) * float(k[b, s2, n2, d]) for d in range(D))
                        tot += max(dot, 0.0) * float(w[b, s1, h])
                    out[b, s1, n2, s2] = tot
    return out


@pytest.mark.parametrize("mode", [0, 3])
def test_indexer_scores_match_brute_force(mode):
    rng = np.random.RandomState(1)
    B, S1, S2, N1, N2, D = 2, 5, 7, 4, 2, 6
    q = rng.randn(B, S1, N1, D); k = rng.randn(B, S2, N2, D); w = rng.randn(B, S1, N1)
    aq, ak = [5, 3], [7, 6]
    got = indexer_scores(q, k, w, aq, ak, mode)
    ref = _brute_scores(q, k, w, aq, ak, mode)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-5, atol=1e-5)


def test_indexer_basis_keys_and_single_head():
    D = 8
    k = np.eye(D)[None, :, None, :]                 # key s2 = e_s2
    q = np.arange(1, D + 1, dtype=np.float64)[None, None, None, :] - 4.5
    w = np.ones((1, 1, 1))
    sc = indexer_scores(q, k, w, [1], [D], 0)[0, 0, 0]
    np.testing.assert_allclose(sc, np.maximum(q[0, 0, 0], 0))


def test_stable_topk_ties_ascending_and_minus1():
    s = np.array([[1.0, 3.0, 3.0, -np.inf, 3.0, 0.5, -np.inf]], np.float32)
    idx, val = stable_topk(s, 6)
    np.testing.assert_array_equal(idx[0], [1, 2, 4, 0, 5, -1])
    assert val[0, -1] == -np.inf
    idx, val = stable_topk(s, 10)   # k > S2 pads with -1
    np.testing.assert_array_equal(idx[0], [1, 2, 4, 0, 5, -1, -1, -1, -1, -1])


def test_stable_topk_matches_torch_stable_sort():
    torch = pytest.importorskip("torch")
    rng = np.random.RandomState(2)
    s = np.round(rng.randn(16, 300) * 4).astype(np.float32)   # many ties
    s[:, 250:] = -np.inf
    s[3, :] = -np.inf
    idx, val = stable_topk(s, 280)
    order = torch.sort(-torch.from_numpy(s), dim=1, stable=True).indices[:, :280].numpy()
    ref_val = np.take_along_axis(s, order, axis=1)
    ref_idx = np.where(ref_val == -np.inf, -1, order)
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_array_equal(val, ref_val)
    # number of -1 entries = max(0, k - visible)
    vis = np.isfinite(s).sum(axis=1)
    np.testing.assert_array_equal((idx == -1).sum(axis=1), np.maximum(0, 280 - vis))


def test_indexer_visible_limit_cases():
    assert visible_limit(3, 4, 10, 0, 10) == 7
    assert visible_limit(3, 4, 2, 0, 10) == 0          # s1 < act_q - act_k
    assert visible_limit(3, 4, 10, 4, 10) == 0          # inactive row
    assert visible_limit(0, 4, 6, 1, 10) == 6


def test_indexer_tnd_equals_bsnd():
    rng = np.random.RandomState(4)
    lens = [3, 5]
    N1, D, K = 4, 8, 4
    qs = [rng.randn(n, N1, D).astype(np.float32) for n in lens]
    ks = [rng.randn(n, 1, D).astype(np.float32) for n in lens]
    ws = [rng.randn(n, N1).astype(np.float32) for n in lens]
    cum = np.cumsum(lens)
    idx, val = lightning_indexer(np.concatenate(qs), np.concatenate(ks), np.concatenate(ws),
                                 cum, cum, layout_query="TND", layout_key="TND",
                                 sparse_count=K, sparse_mode=3, return_value=True,
                                 value_dtype="float32")
    start = 0
    for i, n in enumerate(lens):
        i1, v1 = lightning_indexer(qs[i][None], ks[i][None], ws[i][None], sparse_count=K,
                                   sparse_mode=3, return_value=True, value_dtype="float32")
        np.testing.assert_array_equal(idx[start:start + n], i1[0])
        np.testing.assert_array_equal(val[start:start + n], v1[0])
        start += n


# ---------------------------------------------------------------------------
# KL loss backward
# ---------------------------------------------------------------------------
def _kl_case(rng, B=1, S1=3, S2=6, N1=4, D=8, Dr=4, Ni=3, Di=8, topK=6, full=True):
    q = rng.randn(B, S1, N1, D) * 0.5; k = rng.randn(B, S2, 1, D) * 0.5
    qr = rng.randn(B, S1, N1, Dr) * 0.5; kr = rng.randn(B, S2, 1, Dr) * 0.5
    qi = rng.randn(B, S1, Ni, Di); ki = rng.randn(B, S2, 1, Di)
    w = np.abs(rng.randn(B, S1, Ni))
    si = np.zeros((B, S1, 1, topK), np.int32)
    for b in range(B):
        for s1 in range(S1):
            vis = S2 - S1 + s1 + 1
            n = min(topK, vis)
            si[b, s1, 0, :n] = rng.permutation(vis)[:n]
    scale = 1 / math.sqrt(D + Dr)
    # teacher stats over exactly the selected set: then p sums to one per row
    smax = np.zeros((B, 1, S1, N1)); ssum = np.zeros((B, 1, S1, N1))
    for b in range(B):
        for s1 in range(S1):
            n = min(topK, S2 - S1 + s1 + 1)
            idx = si[b, s1, 0, :n]
            s = (q[b, s1] @ k[b, idx, 0].T + qr[b, s1] @ kr[b, idx, 0].T) * scale
            smax[b, 0, s1] = s.max(1)
            ssum[b, 0, s1] = np.exp(s - s.max(1, keepdims=True)).sum(1)
    return q, k, qr, kr, qi, ki, w, si, smax, ssum, scale


def test_kl_gradients_match_finite_differences():
    rng = np.random.RandomState(7)
    q, k, qr, kr, qi, ki, w, si, smax, ssum, scale = _kl_case(rng)
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, compute_dtype=np.float64)
    np.testing.assert_allclose(r["p"].sum(-1), 1.0, rtol=1e-6)

    def loss(qi_, ki_, w_):
        return float(kl_loss_bwd(q, k, qr, kr, qi_, ki_, w_, si, smax, ssum, scale,
                                 compute_dtype=np.float64)["loss"][0])

    eps = 1e-6
    for which, arr, g in (("qi", qi, r["dQueryIndex"]), ("ki", ki, r["dKeyIndex"]),
                          ("w", w, r["dW"])):
        for idx in list(np.ndindex(arr.shape))[::max(1, arr.size // 15)]:
            a = arr.copy(); a[idx] += eps
            args = {"qi": qi, "ki": ki, "w": w}; args[which] = a
            lp = loss(args["qi"], args["ki"], args["w"])
            a = arr.copy(); a[idx] -= eps
            args[which] = a
            lm = loss(args["qi"], args["ki"], args["w"])
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - g[idx]) < 1e-5 * max(1.0, abs(fd)), (which, idx, fd, g[idx])


def test_kl_invariants():
    rng = np.random.RandomState(8)
    q, k, qr, kr, qi, ki, w, si, smax, ssum, scale = _kl_case(rng, S1=4, S2=9, topK=5)
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, compute_dtype=np.float64)
    assert r["loss"][0] >= 0
    n = np.array([min(5, 9 - 4 + s + 1) for s in range(4)])
    sum_di = r["dI"].sum(-1)[0]
    sum_p = r["p"].sum(-1)[0]
    np.testing.assert_allclose(sum_di, r["softmax_I"].sum(-1)[0] - sum_p, atol=1e-12)
    np.testing.assert_allclose(r["softmax_I"].sum(-1)[0], 1.0, rtol=1e-7)
    # dW_g = sum_k dI * ReLU_g (chain rule through the weighted sum)
    for s1 in range(4):
        idx = si[0, s1, 0, :n[s1]]
        relu = np.maximum(qi[0, s1] @ ki[0, idx, 0].T, 0)
        np.testing.assert_allclose(r["dW"][0, s1], relu @ r["dI"][0, s1, :n[s1]], rtol=1e-10)


def test_kl_zero_when_student_equals_teacher():
    """If every selected key has the same index score and the same teacher
    score, softmax(I) and p are both uniform: KL = 0 and dI = 0."""
    B, S1, S2, N1, D, Ni, Di, topK = 1, 2, 4, 2, 4, 2, 4, 4
    q = np.zeros((B, S1, N1, D)); k = np.ones((B, S2, 1, D))
    qr = np.zeros((B, S1, N1, 4)); kr = np.ones((B, S2, 1, 4))
    qi = np.ones((B, S1, Ni, Di)); ki = np.ones((B, S2, 1, Di)); w = np.ones((B, S1, Ni))
    si = np.tile(np.arange(4, dtype=np.int32), (B, S1, 1, 1))
    smax = np.zeros((B, 1, S1, N1))
    ssum = np.zeros((B, 1, S1, N1))
    for s1 in range(S1):
        ssum[0, 0, s1] = min(topK, S2 - S1 + s1 + 1)
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, 0.5, compute_dtype=np.float64)
    assert abs(r["loss"][0]) < 1e-6
    assert np.abs(r["dI"]).max() < 1e-7


def test_kl_matches_scalar_brute_force():
    rng = np.random.RandomState(9)
    q, k, qr, kr, qi, ki, w, si, smax, ssum, scale = _kl_case(rng, S1=3, S2=5, topK=4)
    si[0, 0, 0, 0] = 9            # out of range entry inside the prefix: clamped
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, compute_dtype=np.float64,
                    dki_oob="clamp")
    B, S1, N1, D = q.shape
    S2, Ni = k.shape[1], qi.shape[2]
    loss = 0.0
    dki = np.zeros_like(ki)
    for s1 in range(S1):
        n = min(4, S2 - S1 + s1 + 1)
        toks = [min(max(int(t), 0), S2 - 1) for t in si[0, s1, 0, :n]]
        I = []
        relus = []
        for t in toks:
            rr = [max(sum(qi[0, s1, g, d] * ki[0, t, 0, d] for d in range(qi.shape[3])), 0.0) for g in range(Ni)]
            relus.append(rr)
            I.append(sum(w[0, s1, g] * rr[g] for g in range(Ni)))
        p = []
        for t in toks:
            acc = 0.0
            for h in range(N1):
                s = (sum(q[0, s1, h, d] * k[0, t, 0, d] for d in range(D)) +
                     sum(qr[0, s1, h, d] * kr[0, t, 0, d] for d in range(qr.shape[3]))) * scale
                acc += math.exp(s - smax[0, 0, s1, h]) / (ssum[0, 0, s1, h] + 1e-8)
            p.append(acc / N1)
        m = max(I)
        z = sum(math.exp(x - m) for x in I)
        sI = [math.exp(x - m) / (z + 1e-8) for x in I]
        for a, b_ in zip(p, sI):
            a2, b2 = max(a, 1e-8), max(b_, 1e-8)
            loss += a2 * (math.log(a2) - math.log(b2))
        for j, t in enumerate(toks):
            dI = sI[j] - p[j]
            for g in range(Ni):
                if relus[j][g] > 0:
                    dki[0, t, 0] += dI * w[0, s1, g] * qi[0, s1, g]
    np.testing.assert_allclose(r["loss"][0], loss, rtol=1e-10)
    np.testing.assert_allclose(r["dKeyIndex"], dki, rtol=1e-10, atol=1e-12)
    # the golden's rule skips the out-of-range target instead of clamping it
    r2 = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, scale, compute_dtype=np.float64,
                     dki_oob="skip")
    assert not np.allclose(r2["dKeyIndex"][0, S2 - 1], r["dKeyIndex"][0, S2 - 1])


# ---------------------------------------------------------------------------
# KL on packed (TND) rows and paged key caches: the compositions agree with
# the BSND oracle where the layouts describe the same problem
# ---------------------------------------------------------------------------
def _kl_bsnd_problem(B=2, S1=5, S2=48, N1=4, D=16, Ni=3, topK=12, seed=5):
    rng = np.random.RandomState(seed)
    f = lambda *s: rng.randn(*s).astype(np.float32)  # noqa: E731
    q, k, qr, kr = f(B, S1, N1, D), f(B, S2, 1, D), f(B, S1, N1, 4), f(B, S2, 1, 4)
    qi, ki = f(B, S1, Ni, 8), f(B, S2, 1, 8)
    w = np.abs(f(B, S1, Ni))
    si = rng.randint(0, S2 + 3, (B, S1, 1, topK)).astype(np.int32)   # some past S2: clamped
    smax = f(B, 1, S1, N1)
    ssum = np.abs(f(B, 1, S1, N1)) + 1.0
    return q, k, qr, kr, qi, ki, w, si, smax, ssum


def test_kl_tnd_oracle_equal_lengths_is_bsnd():
    from oracle.kl import kl_loss_bwd, kl_loss_bwd_tnd
    B, S1, S2 = 2, 5, 48
    q, k, qr, kr, qi, ki, w, si, smax, ssum = _kl_bsnd_problem(B, S1, S2)
    a = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, 0.3, compute_dtype=np.float64)
    flat = lambda x, S: x.reshape(B * S, *x.shape[2:])  # noqa: E731
    b = kl_loss_bwd_tnd(flat(q, S1), flat(k, S2), flat(qr, S1), flat(kr, S2), flat(qi, S1), flat(ki, S2),
                        flat(w, S1), flat(si, S1), smax, ssum, 0.3, np.cumsum([S1] * B), np.cumsum([S2] * B),
                        compute_dtype=np.float64)
    for key in ("dQueryIndex", "dKeyIndex", "dW", "loss"):
        assert np.array_equal(a[key].reshape(-1), b[key].reshape(-1)), key


def test_kl_tnd_oracle_clamps_to_the_batch():
    """A packed batch's out-of-range ids clamp to its own last key, which a
    B = 1 problem of that batch alone reproduces."""
    from oracle.kl import kl_loss_bwd, kl_loss_bwd_tnd
    q, k, qr, kr, qi, ki, w, si, smax, ssum = _kl_bsnd_problem(1, 4, 30)
    lq, lk = [0, 4], [18, 30]
    # batch 1 of the packed problem is the B = 1 problem; batch 0 has keys only
    kk = np.concatenate([np.ones((18, 1, 16), np.float32), k[0]], 0)
    kkr = np.concatenate([np.ones((18, 1, 4), np.float32), kr[0]], 0)
    kki = np.concatenate([np.ones((18, 1, 8), np.float32), ki[0]], 0)
    t = kl_loss_bwd_tnd(q[0], kk, qr[0], kkr, qi[0], kki, w[0], si[0], smax, ssum, 0.3, np.cumsum(lq),
                        np.cumsum(lk), compute_dtype=np.float64)
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, 0.3, compute_dtype=np.float64)
    assert np.array_equal(t["dKeyIndex"][18:], r["dKeyIndex"][0])
    assert np.all(t["dKeyIndex"][:18] == 0)
    assert np.array_equal(t["dQueryIndex"], r["dQueryIndex"][0]) and t["loss"][0] == r["loss"][0]


def test_kl_paged_oracle_matches_bsnd_on_the_depaged_cache():
    from oracle.kl import kl_loss_bwd, kl_loss_bwd_paged
    B, S1, page, mb = 2, 5, 8, 6
    S2 = page * mb
    q, k, qr, kr, qi, ki, w, si, smax, ssum = _kl_bsnd_problem(B, S1, S2)
    rng = np.random.RandomState(9)
    perm = rng.permutation(B * mb + 3)[:B * mb].reshape(B, mb)          # disjoint pages, shuffled
    nblk = B * mb + 3
    caches = []
    for x in (k, kr, ki):
        c = rng.randn(nblk, page, 1, x.shape[-1]).astype(np.float32)   # unused pages hold noise
        for b in range(B):
            for i in range(mb):
                c[perm[b, i]] = x[b, i * page:(i + 1) * page]
        caches.append(c)
    act_k = [S2, S2 - 5]
    p = kl_loss_bwd_paged(q, caches[0], qr, caches[1], qi, caches[2], w, si, smax, ssum, 0.3, perm, act_k,
                          compute_dtype=np.float64)
    r = kl_loss_bwd(q, k, qr, kr, qi, ki, w, si, smax, ssum, 0.3, act_k=act_k, compute_dtype=np.float64)
    for key in ("dQueryIndex", "dW", "loss"):
        assert np.array_equal(p[key], r[key]), key
    for b in range(B):
        for i in range(mb):
            assert np.array_equal(p["dKeyIndex"][perm[b, i]], r["dKeyIndex"][b, i * page:(i + 1) * page])
    unused = sorted(set(range(nblk)) - set(perm.reshape(-1).tolist()))
    assert unused and np.all(p["dKeyIndex"][unused] == 0)
