"""Full-size parity of the backward pair at the benchmarked shape.

cfg5a: SFA backward, B=1, S1=S2=4096, N1=128, D=512+64, topK=2048, causal
indices (row s1 holds min(2048, s1+1) distinct ids from [0, s1], the
benchmark's recipe), bf16, dOut ~ N(0,1), out and statistics from the HIP
forward on the same data.  cfg5b: the KL-loss backward at the same shape with
Nidx1=64, D_idx=128, fp32 weights ~ U(0,1) and the same indices and
statistics.

At this size thousands of query rows hit the same key rows, which is where
the dK / dK_rope / dV scatter and the dKeyIndex reduction do their work.

Checks against the fp32 oracle (the oracle is fed the same bf16 inputs and
the same forward out / statistics, which are inputs of the backward):

* SFA forward: out and statistics on 16 sampled rows.
* SFA backward: dq / dq_rope on 16 sampled rows; dk / dk_rope / dv (and the
  training path's dk + dv) on 32 sampled key rows, including the most-hit
  keys.  A row's contribution to key t depends only on that row's inputs
  and key t (P = exp(s - max) / sum uses the given statistics), so the
  oracle runs each row that hits a sampled key with an index list reduced
  to the sampled keys it hits; its dk at those keys is then the sum over
  exactly the rows whose lists contain them.
* KL backward: every row through the oracle (about 20 s of host work):
  dQueryIndex and dWeights on all rows, dKeyIndex on all key rows, and the
  loss.

Tolerance: the north star's rtol 2e-2 / atol 2e-3 for per-row gradients
(dq, dq_rope, dWeights); for the scatter-added key gradients atol is 2e-3 of
the tensor's largest magnitude (they sum up to ~3500 rows each).  dQi / dKi
at rtol 1e-2 with atol 1e-3 of the largest magnitude, the loss at rtol
1e-3.  dWeights is held to the north star's tolerance here, not the KL
suite's 1e-3: at this shape the index scores reach |I| ~ 250, so softmax(I)
and with it dI = softmax(I) - p carry relative errors of order |I| times
fp32's epsilon in any fp32 evaluation (the fp32 oracle's own dWeights moves
by up to 3e-5 against fp64), and dWeights sums those errors times ReLU
scores of up to ~40.
"""
import math

import numpy as np
import pytest
import torch

from oracle.kl import kl_loss_bwd
from oracle.sfa import sfa_fwd_bsnd
from oracle.sfa_grad import sfa_bwd_bsnd
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

S, N1, D, DR, K = 4096, 128, 512, 64, 2048
NI, DI = 64, 128
SCALE = 1.0 / math.sqrt(D + DR)


def _np(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def cfg5():
    from bench import causal_indices
    import dsa_triton_ascend_amd as dsa
    print("[full-size bwd] building cfg5 inputs", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4242)
    rn = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)  # noqa: E731
    q, qr, k, kr = rn(1, S, N1, D), rn(1, S, N1, DR), rn(1, S, 1, D), rn(1, S, 1, DR)
    do = rn(1, S, N1, D)
    idx, n = causal_indices(S, K, g, dev)
    si = idx.reshape(1, S, 1, K).contiguous()
    qi, ki = rn(1, S, NI, DI), rn(1, S, 1, DI)
    w = torch.rand(1, S, NI, generator=g, device=dev)
    o, smax, ssum = dsa.sparse_flash_attention_triton(q, k, k, si, scale_value=SCALE, query_rope=qr, key_rope=kr,
                                                      sparse_mode=3, return_softmax_lse=True)
    torch.cuda.synchronize()
    t = dict(q=q, qr=qr, k=k, kr=kr, do=do, si=si, qi=qi, ki=ki, w=w, o=o, smax=smax, ssum=ssum)
    host = {name: (_np(v) if v.dtype != torch.int32 else v.cpu().numpy()) for name, v in t.items()}
    return t, host


def _sample_rows():
    rng = np.random.RandomState(5)
    rows = {0, 1, 2047, 2048, 4095} | set(int(x) for x in rng.choice(S, 11, replace=False))
    return sorted(rows)


def _sample_keys():
    rng = np.random.RandomState(6)
    keys = {0, 1, 2, 7, 100, 1000, 2046, 2047, 2048, 3000, 4000, 4093, 4094, 4095}
    while len(keys) < 32:
        keys.add(int(rng.randint(0, S)))
    return sorted(keys)


def test_cfg5_forward_sampled_rows(cfg5):
    _, h = cfg5
    rows = [(0, r) for r in _sample_rows()]
    print(f"[full-size fwd] rows {[r for _, r in rows]}", flush=True)
    ref = sfa_fwd_bsnd(h["q"], h["k"], h["si"], h["qr"], h["kr"], SCALE, [S], [S], 1, 3, True, "float32",
                       positions="kernel", rows=rows)
    sel = [r for _, r in rows]
    assert_close(h["o"][0, sel], ref[0][0, sel], 2e-2, 2e-3, "out")
    assert_close(h["smax"][0, 0, sel], ref[1][0, 0, sel], 2e-2, 2e-3, "softmax_max")
    assert_close(h["ssum"][0, 0, sel], ref[2][0, 0, sel], 2e-2, 2e-3, "softmax_sum")


def _sfa_bwd_gpu(t, merge):
    import dsa_triton_ascend_amd as dsa
    from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad
    if merge:
        res = _sfa_grad(t["q"], t["k"], t["k"], t["si"], t["do"], t["o"], t["smax"], t["ssum"], SCALE, t["qr"],
                        t["kr"], None, None, 1, "BSND", 3, INT64_MAX, INT64_MAX, False, merge_kv=True)
    else:
        res = dsa.sparse_flash_attention_grad_triton(t["q"], t["k"], t["k"], t["si"], t["do"], t["o"], t["smax"],
                                                     t["ssum"], scale_value=SCALE, query_rope=t["qr"],
                                                     key_rope=t["kr"], sparse_mode=3)
    torch.cuda.synchronize()
    return [None if r is None else _np(r) for r in res]


def _oracle_keys(h, keys):
    """The oracle's dk / dv / dk_rope at ``keys``: every row that hits one
    of them, run with its index list reduced to the sampled keys it hits."""
    si = h["si"][0, :, 0, :]
    keyset = np.asarray(keys)
    hit = np.isin(si, keyset)                                  # [S, K]
    rows = np.nonzero(hit.any(axis=1))[0]
    red = np.full((1, S, 1, len(keys)), -1, np.int32)
    for r in rows:
        ks = si[r][hit[r]]
        red[0, r, 0, :ks.size] = ks
    print(f"[full-size bwd] {rows.size} rows hit the {len(keys)} sampled keys", flush=True)
    _, dk, dv, _, dkr = sfa_bwd_bsnd(h["q"], h["k"], red, h["do"], h["o"], h["smax"], h["ssum"], h["qr"], h["kr"],
                                     SCALE, [S], [S], 1, 3, "float32", positions="kernel",
                                     rows=[(0, int(r)) for r in rows], guard_sum=True)
    return dk[0, keys, 0], dv[0, keys, 0], dkr[0, keys, 0]


def _close_scaled(got, exp, what):
    assert_close(got, exp, 2e-2, 2e-3 * max(1.0, float(np.abs(exp).max())), what)


@pytest.mark.parametrize("merge", [False, True], ids=["reference_api", "training_path"])
def test_cfg5a_sfa_bwd(cfg5, merge):
    t, h = cfg5
    print(f"[full-size bwd] cfg5a SFA backward merge={merge}", flush=True)
    dq, dk, dv, dqr, dkr = _sfa_bwd_gpu(t, merge)
    rows = _sample_rows()
    ref = sfa_bwd_bsnd(h["q"], h["k"], h["si"], h["do"], h["o"], h["smax"], h["ssum"], h["qr"], h["kr"], SCALE,
                       [S], [S], 1, 3, "float32", positions="kernel", rows=[(0, r) for r in rows], guard_sum=True)
    assert_close(dq[0, rows], ref[0][0, rows], 2e-2, 2e-3, "dq")
    assert_close(dqr[0, rows], ref[3][0, rows], 2e-2, 2e-3, "dq_rope")
    keys = _sample_keys()
    edk, edv, edkr = _oracle_keys(h, keys)
    if merge:
        assert dv is None
        _close_scaled(dk[0, keys, 0], edk + edv, "dk + dv (training path)")
    else:
        _close_scaled(dk[0, keys, 0], edk, "dk")
        _close_scaled(dv[0, keys, 0], edv, "dv")
    _close_scaled(dkr[0, keys, 0], edkr, "dk_rope")
    assert np.isfinite(dk).all() and np.isfinite(dkr).all()


def test_cfg5b_kl_bwd_all_rows(cfg5):
    import dsa_triton_ascend_amd as dsa
    t, h = cfg5
    print("[full-size bwd] cfg5b KL backward", flush=True)
    dqi, dki, dw, loss = dsa.sparse_lightning_indexer_grad_kl_loss_triton(
        t["q"], t["k"], t["qi"], t["ki"], t["w"], t["si"], t["smax"], t["ssum"], query_rope=t["qr"],
        key_rope=t["kr"], scale_value=SCALE)
    torch.cuda.synchronize()
    dqi, dki, dw, loss = _np(dqi), _np(dki), _np(dw), _np(loss)
    print("[full-size bwd] cfg5b oracle over all rows", flush=True)
    ref = kl_loss_bwd(h["q"], h["k"], h["qr"], h["kr"], h["qi"], h["ki"], h["w"], h["si"], h["smax"], h["ssum"],
                      SCALE)
    errors = []
    for got, exp, rtol, atol, what in (
            (dw, ref["dW"], 2e-2, 2e-3, "dWeights"),
            (dqi, ref["dQueryIndex"], 1e-2, 1e-3 * float(np.abs(ref["dQueryIndex"]).max()), "dQueryIndex"),
            (dki, ref["dKeyIndex"], 1e-2, 1e-3 * float(np.abs(ref["dKeyIndex"]).max()), "dKeyIndex"),
            (loss, ref["loss"], 1e-3, 0.0, "loss")):
        print(f"  {what}: max abs err {np.abs(got - exp).max():.3g}, max |ref| {np.abs(exp).max():.3g}", flush=True)
        try:
            assert_close(got, exp, rtol, atol, what)
        except AssertionError as e:
            errors.append(str(e))
    assert not errors, "; ".join(errors)
