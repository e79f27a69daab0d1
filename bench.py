"""Benchmark of the DSA operator set on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (BASELINE.json metric): sparse flash attention forward at the
DeepSeek-V3.2 decode shape (PA_BSND, block 64, B=32, S1=1, ctx 32768,
N1=128, D=512+64, topK=2048, bf16, sparse_mode 0, scale 1/sqrt(576)), in
TFLOP/s of algorithmic work and % of the bf16 dense MFMA peak.  A "step" is
one forward over the whole batch.  Inputs are resident in HBM before timing;
six independent input sets (KV cache, block table, indices, queries) are
rotated so the 256 MiB Infinity Cache cannot serve the ~75 MB each step
reads.  Timing: HIP events on the launch stream around exactly K steps,
with device synchronisation on both sides.  The roofline object is for the
dominant kernel (sfa_fwd_kernel).  The CPU baseline is the numpy oracle
(tests-only port of the reference golden) on the host.
"""
import argparse
import json
import math
import os
import sys
import time

INT64_MAX = 9223372036854775807  # pre_tokens / next_tokens: no band

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sets", type=int, default=6)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--long-steps", type=int, default=10,
                    help="timed steps of the prefill / backward legs (each step is milliseconds)")
    ap.add_argument("--no-long", action="store_true", help="skip the prefill / backward legs")
    ap.add_argument("--legs", default="prefill,bwd,bwd_merged,kl,dense",
                    help="comma list of the long legs to run (prefill, bwd, bwd_merged, kl, dense)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain copy kernel of known size (for PMC calibration)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# SFA decode workload
# ---------------------------------------------------------------------------
B, N1, D, DR, K, CTX, PAGE = 32, 128, 512, 64, 2048, 32768, 64


def make_decode_sets(nsets, device):
    import torch
    sets = []
    g = torch.Generator(device=device).manual_seed(1234)
    nblk = B * CTX // PAGE
    for _ in range(nsets):
        s = {}
        s["cache"] = torch.randn(nblk, PAGE, 1, D, generator=g, device=device).to(torch.bfloat16)
        s["cache_r"] = torch.randn(nblk, PAGE, 1, DR, generator=g, device=device).to(torch.bfloat16)
        s["q"] = torch.randn(B, 1, N1, D, generator=g, device=device).to(torch.bfloat16)
        s["qr"] = torch.randn(B, 1, N1, DR, generator=g, device=device).to(torch.bfloat16)
        s["bt"] = torch.randperm(nblk, generator=g, device=device).to(torch.int32).reshape(B, CTX // PAGE)
        idx = torch.argsort(torch.rand(B, CTX, generator=g, device=device), dim=1)[:, :K]
        s["si"] = idx.to(torch.int32).reshape(B, 1, 1, K).contiguous()
        sets.append(s)
    return sets


def decode_algorithmic(n_valid):
    """Flops and HBM bytes of one decode step (per-unit figures x units)."""
    flops = 2.0 * N1 * (2 * D + DR) * n_valid
    kv_bytes = n_valid * (D + DR) * 2
    q_bytes = B * N1 * (D + DR) * 2
    o_bytes = B * N1 * D * 2
    idx_bytes = B * K * 4 + B * (CTX // PAGE) * 4
    return flops, kv_bytes + q_bytes + o_bytes + idx_bytes


SETTLE_MS = 200.0


def settle(step, ms=SETTLE_MS):
    """Untimed load before a leg's warmup steps: the GPU's clocks take on the
    order of 100 ms of work to settle (10 warmup steps of the decode are half
    a millisecond; timed after them the decode step is about 14 % slower)."""
    import time
    import torch
    t0 = time.perf_counter()
    i = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        step(i)
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_decode(sets, steps, warmup):
    import torch
    from dsa_triton_ascend_amd import _lib
    lib = _lib.load()
    dev = sets[0]["q"].device
    out = torch.empty(B, 1, N1, D, dtype=torch.bfloat16, device=dev)
    ws_bytes = lib.dsa_sfa_fwd_workspace_size(B, N1, D, K, 1)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    act_k = torch.full((B,), CTX, dtype=torch.int32, device=dev)
    stream = _lib.stream_handle(dev)
    scale = 1.0 / math.sqrt(D + DR)
    nblk = B * CTX // PAGE

    def step(s, strm=stream):
        st = lib.dsa_sfa_fwd(
            s["q"].data_ptr(), s["qr"].data_ptr(), s["cache"].data_ptr(), s["cache_r"].data_ptr(),
            s["si"].data_ptr(), out.data_ptr(), None, None, None, act_k.data_ptr(), s["bt"].data_ptr(),
            B, 1, CTX, N1, D, DR, K, B, nblk * PAGE, CTX // PAGE, PAGE, 1, 0, INT64_MAX, INT64_MAX,
            _lib.LAYOUT["BSND"], _lib.LAYOUT["PA_BSND"], _lib.DTYPE_BF16, scale, 0,
            ws.data_ptr(), ws_bytes, strm)
        if st != 0:
            _lib.check(st, "dsa_sfa_fwd")

    settle(lambda i: step(sets[i % len(sets)]))
    for i in range(warmup):
        step(sets[i % len(sets)])
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(sets[i % len(sets)])
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    # per-step distribution (median / p20 / p80 like the reference harness)
    per = []
    for i in range(min(steps, 50)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        step(sets[i % len(sets)])
        e1.record()
        e1.synchronize()
        per.append(e0.elapsed_time(e1))
    per.sort()
    # the same step captured once in a HIP graph (both kernels) and replayed:
    # K replays back to back, no host launch work between them
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(sets[0], torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(sets[0], torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    g0 = torch.cuda.Event(enable_timing=True)
    g1 = torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(steps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    graph_ms = g0.elapsed_time(g1) / steps
    del graph
    return total_ms / steps, per, graph_ms


def cpu_baseline_decode(sets):
    """numpy oracle over the full decode batch of one input set (host cores)."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_info
        cores = max(int(i.get("num_threads", 1)) for i in threadpool_info()) if threadpool_info() else 1
    except Exception:
        cores = len(os.sched_getaffinity(0))
    from oracle.sfa import sfa_fwd_bsnd
    s = sets[0]
    si = s["si"].cpu().numpy()
    bt = s["bt"].cpu().numpy()
    cache = s["cache"].reshape(-1, D)
    cache_r = s["cache_r"].reshape(-1, DR)
    q = s["q"].float().cpu().numpy()
    qr = s["qr"].float().cpu().numpy()
    rows = list(range(B))
    # gather each row's selected KV (the reference de-pages on the host too)
    ks, krs = [], []
    for b in rows:
        toks = si[b, 0, 0]
        phys = bt[b, toks // PAGE].astype(np.int64) * PAGE + toks % PAGE
        import torch
        pt = torch.from_numpy(phys).to(cache.device)
        ks.append(cache[pt].float().cpu().numpy())
        krs.append(cache_r[pt].float().cpu().numpy())
    idx = np.arange(K, dtype=np.int32).reshape(1, 1, 1, K)
    scale = 1.0 / math.sqrt(D + DR)
    # the whole batch, repeated until at least ~10 s of host work is timed
    reps = 0
    t0 = time.perf_counter()
    while True:
        for b in rows:
            sfa_fwd_bsnd(q[b:b + 1], ks[b][None, :, None, :], idx, qr[b:b + 1],
                         krs[b][None, :, None, :], scale, [1], [K], 1, 0, True, "bfloat16",
                         positions="kernel")
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= 10.0:
            break
    flops, _ = decode_algorithmic(B * K)
    return {"value": reps * flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"numpy oracle (port of sparse_flash_attention_numpy.py) over the full "
                      f"decode batch of one input set ({B} rows x {K} tokens x {N1} heads), "
                      f"repeated {reps} times, {dt:.1f} s"}


# ---------------------------------------------------------------------------
# lightning indexer decode workload (secondary metric: us/query at 32K ctx)
# ---------------------------------------------------------------------------
LI_B, LI_S2, LI_N1, LI_D, LI_K = 32, 32768, 64, 128, 2048


def make_li_sets(nsets, device):
    import torch
    g = torch.Generator(device=device).manual_seed(4321)
    sets = []
    for _ in range(nsets):
        sets.append({
            "q": torch.randn(LI_B, 1, LI_N1, LI_D, generator=g, device=device).to(torch.bfloat16),
            "k": torch.randn(LI_B, LI_S2, 1, LI_D, generator=g, device=device).to(torch.bfloat16),
            "w": torch.rand(LI_B, 1, LI_N1, generator=g, device=device),
        })
    return sets


def li_algorithmic():
    """Flops and HBM bytes of one indexer decode step (all keys visible)."""
    pairs = LI_B * LI_S2
    flops = 2.0 * LI_N1 * LI_D * pairs
    nbytes = pairs * LI_D * 2 + LI_B * LI_N1 * (LI_D * 2 + 4) + LI_B * LI_K * 4
    return flops, nbytes


def time_li(sets, steps, warmup):
    import torch
    from dsa_triton_ascend_amd import _lib
    lib = _lib.load()
    dev = sets[0]["q"].device
    idx = torch.empty(LI_B, 1, 1, LI_K, dtype=torch.int32, device=dev)
    ws_bytes = lib.dsa_li_fwd_workspace_size(LI_B, 1, LI_S2)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    def step(s):
        st = lib.dsa_li_fwd(s["q"].data_ptr(), s["k"].data_ptr(), s["w"].data_ptr(), None, None,
                            idx.data_ptr(), None, LI_B, 1, LI_S2, LI_N1, 1, LI_D, LI_K, LI_B,
                            LI_B * LI_S2, 3, _lib.LAYOUT["BSND"], _lib.LAYOUT["BSND"], _lib.DTYPE_BF16,
                            _lib.DTYPE_FP32, 0, ws.data_ptr(), ws_bytes, stream)
        if st != 0:
            _lib.check(st, "dsa_li_fwd")

    settle(lambda i: step(sets[i % len(sets)]))
    for i in range(warmup):
        step(sets[i % len(sets)])
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(sets[i % len(sets)])
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# ---------------------------------------------------------------------------
# prefill forward (cfg4) and the backward pair (cfg5a / cfg5b): reported
# beside the headline, each in TFLOP/s of algorithmic work
# ---------------------------------------------------------------------------
def causal_indices(S, K, g, device):
    """Row s1 holds min(K, s1+1) distinct uniform ids from [0, s1], sorted,
    -1-padded to K (the prefill config's index recipe)."""
    import torch
    r = torch.rand(S, S, generator=g, device=device)
    ar = torch.arange(S, device=device)
    r[ar[None, :] > ar[:, None]] = 2.0
    idx = torch.sort(torch.argsort(r, dim=1)[:, :K], dim=1).values.to(torch.int32)
    del r
    nval = torch.clamp(ar + 1, max=K)
    idx[torch.arange(K, device=device)[None, :] >= nval[:, None]] = -1
    return idx, int(nval.sum())


def time_call(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def leg(metric, workload, flops, ms, n):
    """A secondary leg: algorithmic flops over the step time.  These legs are
    MFMA-bound by their arithmetic intensity (the gathered rows they re-read
    are served from L2 / MALL), so their roofline is the bf16 MFMA peak; the
    measured HBM bytes of each kernel are in profiles/."""
    tf = flops / (ms * 1e-3) / 1e12
    return {"metric": metric, "value": round(tf, 2), "unit": "TFLOP/s", "higher_is_better": True,
            "ms_per_step": round(ms, 4), "pct_of_bf16_peak": round(100.0 * tf / PEAK_BF16_TFLOPS, 3),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_BF16_TFLOPS, 4)},
            "algorithmic_flops": int(flops), "valid_pairs": n, "config": {"workload": workload}}


def long_legs(dev, steps, legs=("prefill", "bwd", "bwd_merged", "kl", "dense")):
    import torch
    import dsa_triton_ascend_amd as dsa
    out = {}
    g = torch.Generator(device=dev).manual_seed(42)
    rn = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)  # noqa: E731
    scale = 1.0 / math.sqrt(D + DR)
    # cfg4: prefill, TND one sequence T=8192, mode 3, stats returned
    T = 8192
    q, qr, k, kr = rn(T, N1, D), rn(T, N1, DR), rn(T, 1, D), rn(T, 1, DR)
    idx, n = causal_indices(T, K, g, dev)
    si = idx.reshape(T, 1, K).contiguous()
    cu = [T]

    def fwd_tnd():
        return dsa.sparse_flash_attention_triton(q, k, k, si, scale_value=scale, actual_seq_lengths_query=cu,
                                                 actual_seq_lengths_kv=cu, query_rope=qr, key_rope=kr,
                                                 layout_query="TND", layout_kv="TND", sparse_mode=3,
                                                 return_softmax_lse=True)
    if "prefill" in legs:
        ms = time_call(fwd_tnd, steps, 2)
        out["sfa_fwd_prefill"] = leg("SFA fwd TFLOP/s (prefill)",
                                   "sfa_fwd prefill: TND one sequence T=8192, N1=128, D=512+64, topK=2048 "
                                   "causal, sparse_mode 3, stats returned", 2.0 * N1 * (2 * D + DR) * n, ms, n)
    del q, qr, k, kr, idx, si
    torch.cuda.empty_cache()
    # cfg5a / cfg5b: backward pair at S=4096
    S = 4096
    q, qr, k, kr = rn(1, S, N1, D), rn(1, S, N1, DR), rn(1, S, 1, D), rn(1, S, 1, DR)
    do = rn(1, S, N1, D)
    idx, n = causal_indices(S, K, g, dev)
    si = idx.reshape(1, S, 1, K).contiguous()
    o, smax, ssum = dsa.sparse_flash_attention_triton(q, k, k, si, scale_value=scale, query_rope=qr, key_rope=kr,
                                                      sparse_mode=3, return_softmax_lse=True)

    def bwd():
        return dsa.sparse_flash_attention_grad_triton(q, k, k, si, do, o, smax, ssum, scale_value=scale,
                                                      query_rope=qr, key_rope=kr, sparse_mode=3)
    if "bwd" in legs:
        ms = time_call(bwd, steps, 2)
        out["sfa_bwd"] = leg("SFA bwd TFLOP/s", "sfa_bwd: BSND B=1, S1=S2=4096, N1=128, D=512+64, topK=2048 "
                           "causal, sparse_mode 3, bf16", 2.0 * N1 * (3 * (D + DR) + 2 * D) * n, ms, n)
    # the training path (autograd): the shared-latent gradient dk + dv in one output
    from dsa_triton_ascend_amd.sparse_flash_attention import INT64_MAX
    from dsa_triton_ascend_amd.sparse_flash_attention_grad import _sfa_grad

    def bwd_merged():
        return _sfa_grad(q, k, k, si, do, o, smax, ssum, scale, qr, kr, None, None, 1, "BSND", 3, INT64_MAX,
                         INT64_MAX, False, merge_kv=True)
    if "bwd_merged" in legs:
        ms = time_call(bwd_merged, steps, 2)
        out["sfa_bwd_merged"] = leg("SFA bwd TFLOP/s (training path, d_key = dk + dv)",
                                  "sfa_bwd as called by the autograd Function (MLA absorb: one key gradient dk + dv): "
                                  "BSND B=1, S1=S2=4096, N1=128, D=512+64, topK=2048 causal, sparse_mode 3, bf16",
                                  2.0 * N1 * (3 * (D + DR) + 2 * D) * n, ms, n)
    NI, DI = 64, 128
    qi, ki = rn(1, S, NI, DI), rn(1, S, 1, DI)
    w = torch.rand(1, S, NI, generator=g, device=dev)

    def kl():
        return dsa.sparse_lightning_indexer_grad_kl_loss_triton(q, k, qi, ki, w, si, smax, ssum, query_rope=qr,
                                                                key_rope=kr, scale_value=scale)
    if "kl" in legs:
        ms = time_call(kl, steps, 2)
    if "kl" in legs:
        out["kl_bwd"] = leg("indexer KL-loss bwd TFLOP/s",
                          "sparse_lightning_indexer_grad_kl_loss: B=1, S1=S2=4096, N1=128, D=512+64, Nidx1=64, "
                          "D_idx=128, topK=2048 causal, bf16 (fp32 weights), stats from the SFA forward",
                          n * (3 * 2 * NI * DI + 2 * N1 * (D + DR) + 2 * NI), ms, n)
    del si, o, do
    torch.cuda.empty_cache()
    # dense warm-up stage at the same shape: every causal key, teacher stats of
    # the dense causal forward [B, N2, S1, G]
    if "dense" not in legs:
        return out
    dsmax, dssum = dense_stats(q, qr, k, kr, scale)

    def dense():
        return dsa.dense_loss_backward_triton(q, k, qi, ki, w, dsmax, dssum, scale_value=scale, query_rope=qr,
                                              key_rope=kr)
    ms = time_call(dense, steps, 2)
    nd = S * (S + 1) // 2
    out["dense_kl_bwd"] = leg("dense indexer KL-loss bwd TFLOP/s",
                              "dense_loss_backward (warm-up stage, index LSE computed inside): B=1, S1=S2=4096, "
                              "N1=128, N2=1, D=512+64, Nidx1=64, D_idx=128, all causal keys, bf16 (fp32 weights)",
                              nd * (3 * 2 * NI * DI + 2 * N1 * (D + DR) + 2 * NI), ms, nd)
    return out


def dense_stats(q, qr, k, kr, scale, rows=256):
    """Softmax max / sum of the dense causal attention, [1, 1, S, N1] fp32."""
    import torch
    S = q.shape[1]
    kk = torch.cat([k[0, :, 0], kr[0, :, 0]], -1).float()                     # [S, D+Dr]
    smax = torch.empty(1, 1, S, q.shape[2], device=q.device)
    ssum = torch.empty_like(smax)
    ar = torch.arange(S, device=q.device)
    for r0 in range(0, S, rows):
        qq = torch.cat([q[0, r0:r0 + rows], qr[0, r0:r0 + rows]], -1).float()  # [r, N1, D+Dr]
        sc = torch.matmul(qq, kk.T) * scale                                      # [r, N1, S]
        sc.masked_fill_((ar[None, :] > ar[r0:r0 + rows, None])[:, None, :], float("-inf"))
        m = sc.amax(-1)
        smax[0, 0, r0:r0 + rows] = m
        ssum[0, 0, r0:r0 + rows] = torch.exp(sc - m[..., None]).sum(-1)
        del sc
    return smax, ssum


def stream_read_rate(device, nbytes=1 << 30, launches=10):
    """GB/s of the library's streaming-read calibration kernel (each byte of
    a 1 GiB buffer read once per launch, 16-byte loads), plain and
    non-temporal: the read rate HBM-bound kernels can reach on this device,
    next to the published 8 TB/s peak."""
    import torch
    from dsa_triton_ascend_amd import _lib
    lib = _lib.load()
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    stream = _lib.stream_handle(device)
    out = {}
    for name, nt in (("plain", 0), ("nontemporal", 1)):
        for _ in range(3):
            _lib.check(lib.dsa_calib_stream_read(buf.data_ptr(), nbytes, nt, None, stream), "calib")
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(launches):
            _lib.check(lib.dsa_calib_stream_read(buf.data_ptr(), nbytes, nt, None, stream), "calib")
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(nbytes * launches / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del buf
    torch.cuda.empty_cache()
    return out


def measured_traffic(name="sfa_fwd_decode_traffic"):
    """HBM bytes per step from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (scaled by a copy kernel of known size), or None."""
    path = os.path.join(ROOT, "profiles", name + ".json")
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes_per_step"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    # the indexer leg first, in the process's first allocations: after the
    # decode leg's ~7 GB of inputs have been allocated and freed, the same
    # indexer step measures about 12 % slower (its streaming reads then run
    # over fragmented mappings)
    stream_read = stream_read_rate(dev)  # the device's streaming-read rate, fresh memory
    li_sets = make_li_sets(max(2, min(args.sets, 4)), dev)
    n_li_sets = len(li_sets)
    li_ms = time_li(li_sets, args.steps, args.warmup)
    del li_sets
    torch.cuda.empty_cache()
    sets = make_decode_sets(args.sets, dev)
    torch.cuda.synchronize()
    ms, per, graph_ms = time_decode(sets, args.steps, args.warmup)
    n_valid = B * K
    flops, nbytes = decode_algorithmic(n_valid)
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    attainable = min(PEAK_BF16_TFLOPS, flops / nbytes * PEAK_HBM_GBS / 1e3)
    result = {
        "metric": "SFA fwd TFLOP/s (decode, DeepSeek-V3.2 shape)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": SETTLE_MS,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn, 6 rotating input sets)",
        "config": {"workload": "sfa_fwd decode: PA_BSND block 64, B=32, S1=1, ctx 32768, "
                               "N1=128, D=512+64, topK=2048, sparse_mode 0",
                   "input_sets": args.sets},
        "pct_of_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 3),
        "pct_of_attainable_roofline": round(100.0 * tflops / attainable, 2),
        "per_step_ms": {"median": round(per[len(per) // 2], 5), "p20": round(per[len(per) // 5], 5),
                        "p80": round(per[4 * len(per) // 5], 5)},
        "hip_graph": {"ms_per_step": round(graph_ms, 5), "value": round(flops / (graph_ms * 1e-3) / 1e12, 2),
                      "note": "the step captured once in a HIP graph and replayed K times (input set 0)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "sfa_fwd_ds_kernel (64 heads, 4 token splits) + sfa_combine_kernel (one step)",
                     "algorithmic_bytes_per_launch": int(nbytes),
                     "algorithmic_flops_per_launch": int(flops),
                     "mfma_tflops": round(tflops, 2),
                     "mfma_frac_of_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4)},
    }
    if args.calib_copy:
        # a plain streaming kernel of known traffic (256 MiB read + 256 MiB
        # written) with a distinctive name, to scale FETCH_SIZE / WRITE_SIZE
        src = torch.zeros(1 << 26, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
    # the device's streaming-read rate (plain and non-temporal loads)
    result["stream_read_GBps"] = stream_read
    # secondary metric: lightning indexer, us/query at 32K context
    del sets
    torch.cuda.empty_cache()
    li_flops, li_bytes = li_algorithmic()
    li_gbs = li_bytes / (li_ms * 1e-3) / 1e9
    result["lightning_indexer"] = {
        "metric": "lightning_indexer us/query at 32K ctx (decode)",
        "value": round(li_ms * 1e3 / LI_B, 4), "unit": "us/query", "higher_is_better": False,
        "ms_per_step": round(li_ms, 5),
        "config": {"workload": "lightning_indexer decode: BSND, B=32, S1=1, S2=32768, N1=64, N2=1, "
                               "D=128, k=2048, sparse_mode 3, bf16 q/k, fp32 weights",
                   "input_sets": n_li_sets},
        "roofline": {"bound": "hbm", "achieved": round(li_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(li_gbs / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic("lightning_indexer_decode_traffic"),
                     "kernel": "li_score_kernel + li_topk_kernel (one step)",
                     "algorithmic_bytes_per_launch": int(li_bytes),
                     "algorithmic_flops_per_launch": int(li_flops)},
    }
    if not args.no_long:
        result.update(long_legs(dev, args.long_steps, tuple(args.legs.split(","))))
        torch.cuda.empty_cache()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_decode(make_decode_sets(1, dev))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
