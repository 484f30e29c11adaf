"""Benchmark of the Maba v2 hot path on one MI355X.

Headline (BASELINE.json ``metric``): DGDA chunked prefill throughput at
T = 32k: B=4, H=10, T=32768, d_k=d_v=64, bf16 q/k/v,
fp32 per-token gates (stride-0 broadcast over channels), fp32 state, output in
q's dtype (bf16).  One step = one ``dgda_prefill`` over the whole batch with
inputs resident in HBM.  ``value`` = B*T / step time (tokens/s).

Also reported in the same JSON line:
  * ``roofline``   -- the DGDA prefill op (three launches: segment aggregate,
                      zero-start output, fix-up output) against HBM: algorithmic
                      bytes per step / step time (HIP events on the launch
                      stream), plus the bf16-MFMA fraction of the algorithmic
                      flops;
  * ``cpu_baseline`` -- the C/OpenMP restatement of the reference CPU chunked
                      algorithm (oracle/dgda_chunked.c) on the same workload, on
                      the host cores;
  * ``decode``     -- BASELINE configs 2b-4: the B=64 DGDA decode microbench
                      (10,000 steps), centroid pooling of the 1M cache, the
                      DG-Indexer decode scoring + top-32 at 1M context and the
                      fused MABA-SA decode step at 1M context (us/step and HBM
                      GB/s each);
  * ``rows``       -- the DGDA prefill with per-channel gates (the layer's gate
                      layout) at the config-2 shape and the causal prefill
                      index_topk.
Each decode / rows entry carries its own ``cpu_baseline``: the oracle timed on
the host on a bounded sample of that workload (the sample is named).

``python bench.py --gpus N --steps K --warmup W``; only N = 1 is supported.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "maba-v2-architecture_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")
TRAFFIC_SOURCE = ("profiles/traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE passes scaled by a device copy's "
                  "readings (profiles/hbm_traffic_pmc.txt)")


def measured_traffic(key):
    """HBM bytes per call of a workload from the committed counter runs, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as fh:
        return json.load(fh).get(key)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true", help="do not time the CPU baseline")
    ap.add_argument("--skip-decode", action="store_true", help="do not run the decode benchmarks")
    ap.add_argument("--only-prefill", action="store_true", help="time only the DGDA prefill step (for profiling)")
    ap.add_argument("--only-decode", action="store_true", help="run only the decode benchmarks (for profiling)")
    ap.add_argument("--only-rows", action="store_true",
                    help="run only the secondary row benchmarks: per-channel-gate prefill, prefill top-k (for profiling)")
    ap.add_argument("--only-model", action="store_true", help="run only the config-5 full-model decode")
    ap.add_argument("--row", default=None,
                    help="with --only-rows: a comma-separated subset of the row groups dgda, prologue, topk, "
                         "superposition, prefill_attention, layer_decode, model (for profiling)")
    ap.add_argument("--model-batch", type=int, default=16)
    ap.add_argument("--model-prefill", type=int, default=131072)
    ap.add_argument("--model-steps", type=int, default=256)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 256 MiB device-to-device copy (calibrates FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def time_op(fn, steps: int, warmup: int):
    """Mean ms per call over ``steps`` calls, HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall


def graph_time(fn, reps: int, check: bool = True):
    """Mean ms per replay of ``fn`` captured in a HIP graph (events on the replay stream).

    With ``check``, the graph's outputs of the first replay must equal an eager call's
    outputs (``fn`` must then be a pure function of its inputs)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            ref = fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = fn()
    g.replay()
    torch.cuda.synchronize()
    if check and not torch.equal(res, ref):
        raise RuntimeError("graph replay differs from the eager result")
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def dgda_prefill_case(dev, B=4, H=10, T=32768, d=64, seed=0):
    import torch
    import torch.nn.functional as F
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1).to(dev, torch.bfloat16)
    k = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1).to(dev, torch.bfloat16)
    v = torch.randn(B, H, T, d, generator=g).to(dev, torch.bfloat16)
    la = (-F.softplus(torch.randn(B, H, T, 1, generator=g) + 2.0)).to(dev)
    beta = torch.sigmoid(torch.randn(B, H, T, 1, generator=g)).to(dev)
    return dict(q=q, k=k, v=v, log_alpha=la.expand(B, H, T, d), b=beta.expand(B, H, T, d),
                w=beta.expand(B, H, T, d))


def prefill_bytes(B, H, T, d):
    """Algorithmic HBM bytes of one prefill step: q,k,v bf16 + two per-token fp32
    gates (log-decay, beta) + bf16 output + fp32 final state."""
    return B * H * T * (3 * d * 2 + 2 * 4 + d * 2) + B * H * d * d * 4


def prefill_flops(B, H, T, d, C=64):
    """Chunked-algorithm flops, (8 C^2 d + 6 C d^2) per (b, h, chunk)."""
    return B * H * (T // C) * (8 * C * C * d + 6 * C * d * d)


def cpu_baseline(B=4, H=10, T=32768, d=64, min_seconds=10.0):
    """The C/OpenMP restatement of the reference CPU chunked prefill (oracle/dgda_chunked.c,
    cpu_dgda.py:33-197 streamed per chunk) on the config-2 shape in fp32: 2 untimed
    repeats, then repeats until ``min_seconds`` have elapsed (benchmark.py:684-745 method)."""
    import numpy as np
    from oracle import dgda_c
    dgda_c.build()
    r = np.random.default_rng(0)
    q = r.standard_normal((B, H, T, d), dtype=np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = r.standard_normal((B, H, T, d), dtype=np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = r.standard_normal((B, H, T, d), dtype=np.float32)
    la = (-np.log1p(np.exp(r.standard_normal((B, H, T, 1), dtype=np.float32) + 2))).astype(np.float32)
    be = (1 / (1 + np.exp(-r.standard_normal((B, H, T, 1), dtype=np.float32)))).astype(np.float32)
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    ncpu = os.cpu_count() or 1
    threads = min(ncpu, omp if omp > 0 else ncpu, B * H)

    def run():
        dgda_c.dgda_prefill_chunked_c(q, k, v, la, be, be, chunk_size=64, nthreads=threads)

    for _ in range(2):
        run()
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds and reps >= 3:
            break
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in fh if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": reps * B * T / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"dgda_prefill config 2 shape B={B} H={H} T={T} d={d}, fp32, chunk 64, "
                      f"{reps} timed repeats in {dt:.1f} s after 2 warm-ups, oracle/dgda_chunked.c (OpenMP over b*h)",
            "host": {"cpu_model": cpu_model, "os_cpu_count": ncpu, "omp_num_threads": omp or None}}


def _timed(fn, min_seconds: float):
    """(repeats, seconds) of ``fn`` after one untimed call, repeated until ``min_seconds``."""
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            return reps, dt


def cpu_anchor_config1(min_seconds: float = 5.0):
    """BASELINE config 1 on the host cores, the required CPU anchor: DGDA forward at B=1,
    H=10, T=2048, d=64 in fp32 through the package's ``cpu`` backend (the chunked form of the
    reference's CPU kernels, kernels/cpu_dgda.py; chunk 16, adaptive inversion) with the
    config's distributions: q, k ~ N(0,1) L2-normalised, v ~ N(0,1), beta = sigmoid(N(0,1)),
    log alpha = -softplus(N(0,1) + 2) per token, zero initial state."""
    import torch
    import torch.nn.functional as F
    from maba_sparse.kernels.cpu_dgda import cpu_dgda_prefill
    B, H, T, d = 1, 10, 2048, 64
    g = torch.Generator().manual_seed(0)
    q = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1)
    v = torch.randn(B, H, T, d, generator=g)
    be = torch.sigmoid(torch.randn(B, H, T, 1, generator=g)).expand(B, H, T, d)
    la = (-F.softplus(torch.randn(B, H, T, 1, generator=g) + 2)).expand(B, H, T, d)
    reps, dt = _timed(lambda: cpu_dgda_prefill(q, k, v, b=be, w=be, log_alpha=la, chunk_size=16), min_seconds)
    return {"value": reps * B * T / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "config": "BASELINE config 1: DGDA forward B=1 H=10 T=2048 d_k=d_v=64 fp32, zero initial state",
            "sample": f"the full config, {reps} repeats in {dt:.1f} s after one warm-up; the package's cpu "
                      f"backend (maba_sparse/kernels/cpu_dgda.py, chunk 16, adaptive inversion) on torch's "
                      f"intra-op threads"}


def cpu_row_baselines(min_seconds: float = 2.0):
    """The CPU baselines beside the secondary rows, on the host cores: the package's torch-CPU
    ops (the ``cpu`` backend: chunked DGDA, the reference ops for the indexer and MABA-SA) at
    the rows' full shapes where that fits a few seconds, otherwise on a stated sample (the
    dense prefill attention: a chunk of queries)."""
    import torch
    import torch.nn.functional as F
    from maba_sparse.kernels import common as C
    from maba_sparse.kernels.cpu_dgda import cpu_dgda_prefill, cpu_dgda_step
    out = {}
    nthr = torch.get_num_threads()
    g = torch.Generator().manual_seed(7)
    # DGDA decode step, B=64 H=10 d=64, fp32 (cpu backend's step)
    B, H, d = 64, 10, 64
    q = F.normalize(torch.randn(B, H, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, H, d, generator=g), dim=-1)
    v = torch.randn(B, H, d, generator=g)
    la = (-F.softplus(torch.randn(B, H, 1, generator=g) + 2)).expand(B, H, d)
    be = torch.sigmoid(torch.randn(B, H, 1, generator=g)).expand(B, H, d)
    S = torch.zeros(B, H, d, d)
    reps, dt = _timed(lambda: cpu_dgda_step(q, k, v, b=be, w=be, state=S, log_alpha=la), min_seconds)
    out["dgda_step_B64"] = {"value": dt / reps * 1e6, "unit": "us/step", "cores": nthr, "kind": "port",
                            "sample": f"the full B=64 step in fp32, {reps} repeats in {dt:.1f} s; "
                                      f"maba_sparse/kernels/cpu_dgda.py cpu_dgda_step"}
    # DG-Indexer decode at 1M context: B=8, 10 heads, 15,625 centroids, d=128, top-32 (full config 3 step)
    B, Hq, nb, dc = 8, 10, 15625, 128
    qi = torch.randn(B, Hq, dc, generator=g)
    cent = torch.randn(B, nb, dc, generator=g)
    reps, dt = _timed(lambda: C.ref_index_topk_decode(qi, cent, lambda_dist=0.1, top_k=32), min_seconds)
    out["index_topk_decode_1M"] = {"value": dt / reps * 1e6, "unit": "us/step", "cores": nthr, "kind": "port",
                                   "sample": f"the full config-3 step in fp32, {reps} repeats in {dt:.1f} s; "
                                             f"kernels/common.py ref_index_topk_decode (torch)"}
    del cent
    # MABA-SA decode at 1M context: one batch element of config 4 at full length (scaled by 8)
    Bs, L, H = 1, 1_000_000, 10
    c = torch.randn(Bs, L, dc, generator=g)
    hca = C.ref_hca_pool(c, pool=64)
    ql = torch.randn(Bs, H, dc, generator=g) * 0.1
    idx = torch.stack([torch.randperm(L // 64, generator=g)[:32] for _ in range(H)]).unsqueeze(0)
    gate = torch.randn(Bs, 3, generator=g)
    reps, dt = _timed(lambda: C.ref_maba_sa_decode(ql, c, hca, idx, gate, L=L, scale=0.125), min_seconds)
    out["maba_sa_decode_1M"] = {"value": dt / reps * 1e6 * 8, "unit": "us/step", "cores": nthr, "kind": "port",
                                "sample": f"one of the 8 batch elements of config 4 (L=1M, H=10, d_c=128, per-head "
                                          f"top-32 rows) in fp32, {reps} repeats in {dt:.1f} s, times 8; "
                                          f"kernels/common.py ref_maba_sa_decode (torch)"}
    del c, hca
    # DGDA prefill with per-channel gates: B=1 H=10 T=2048 of the config-2 shape, fp32 chunked
    B, H, T = 1, 10, 2048
    q = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1)
    v = torch.randn(B, H, T, d, generator=g)
    la = -F.softplus(torch.randn(B, H, T, d, generator=g) + 2)
    be = torch.sigmoid(torch.randn(B, H, T, d, generator=g))
    reps, dt = _timed(lambda: cpu_dgda_prefill(q, k, v, b=be, w=be, log_alpha=la, chunk_size=16), min_seconds)
    out["dgda_prefill_per_channel_gates"] = {
        "value": reps * B * T / dt, "unit": "tokens/s", "cores": nthr, "kind": "port",
        "sample": f"B=1 H=10 T=2048 d=64 of the config-2 shape with per-channel fp32 gates, {reps} repeats in "
                  f"{dt:.1f} s; maba_sparse/kernels/cpu_dgda.py cpu_dgda_prefill (chunk 16)"}
    # DGDA layer prologue: B=1, 8,192 of the 32,768 tokens, C=640, fp32 (the torch reference op)
    Tp, Cp = 8192, 640
    xs = [torch.randn(1, Tp, Cp, generator=g) for _ in range(6)]
    wsp = [torch.randn(Cp, 1, 4, generator=g) * 0.3 for _ in range(3)]
    reps, dt = _timed(lambda: C.ref_dgda_prologue(xs, wsp, None, n_heads=10, with_alpha=False), min_seconds)
    out["dgda_layer_prologue"] = {"value": dt / reps * 1e6 * (4 * 32768 / Tp), "unit": "us/call", "cores": nthr,
                                  "kind": "port",
                                  "sample": f"B=1, 8,192 of the 32,768 tokens (C=640) in fp32, {reps} repeats in "
                                            f"{dt:.1f} s, scaled by 16 to the B=4 call; kernels/common.py "
                                            f"ref_dgda_prologue (torch)"}
    del xs
    # MABA-SA prefill streams: the package's torch op (dense masks, fp32, torch's intra-op threads)
    # on the last 64 of the 32,768 queries of all ten heads, scaled by 512 query chunks
    Lp, dhp, Kp, Hp, Qp = 32768, 64, 32, 10, 64
    tg = torch.Generator().manual_seed(7)
    qp1 = torch.randn(1, Hp, Qp, dhp, generator=tg)
    kp1, vp1 = torch.randn(1, Hp, Lp, dhp, generator=tg), torch.randn(1, Hp, Lp, dhp, generator=tg)
    khp, vhp = torch.randn(1, Hp, Lp // 64, dhp, generator=tg), torch.randn(1, Hp, Lp // 64, dhp, generator=tg)
    idxp = torch.randint(0, Lp // 64, (1, Qp, Kp), generator=tg)
    gp = torch.randn(1, Qp, 3, generator=tg)
    reps, dt = _timed(lambda: C.ref_maba_sa_prefill(qp1, kp1, vp1, khp, vhp, None, idxp, gp, scale=0.125), min_seconds)
    out["maba_sa_prefill_32k"] = {"value": dt / reps * 1e3 * (Lp / Qp), "unit": "ms/call", "cores": nthr,
                                  "kind": "port",
                                  "sample": f"the last {Qp} of 32,768 queries of all {Hp} heads (random top-{Kp} "
                                            f"rows), {reps} repeats in {dt:.1f} s, scaled by {Lp // Qp} query "
                                            f"chunks; kernels/common.py ref_maba_sa_prefill (torch fp32)"}
    del kp1, vp1
    # config 5 on the host: the same 101M stack in fp32 through the dispatcher's torch reference
    # ops (the reference's own CPU path), B=1, a 256-token prefill, then 8 greedy steps
    import torch
    from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
    torch.manual_seed(0)
    cm = MabaSparseForCausalLM(get_101m_config()).init_normal(0.02).eval()
    cids = torch.randint(0, 32768, (1, 256))
    marks = []
    t0 = time.perf_counter()
    cm.generate_greedy(cids, 9, on_prefill_done=lambda: marks.append(time.perf_counter()))
    t1 = time.perf_counter()
    out["model_decode_config5"] = {"value": (t1 - marks[0]) / 8 * 1e3, "unit": "ms/token", "cores": torch.get_num_threads(),
                                   "kind": "port",
                                   "sample": f"B=1, 256-token prefill ({marks[0] - t0:.1f} s), then 8 greedy steps; the "
                                             f"same stack in fp32 on the host through the torch reference ops"}
    del cm
    # causal prefill index_topk: the 32,768 query rows against 512 centroids, d=128 (full row shape)
    qp = torch.randn(1, 32768, dc, generator=g)
    cp = torch.randn(1, 512, dc, generator=g)
    reps, dt = _timed(lambda: C.ref_index_topk(qp, cp, lambda_dist=0.5, top_k=32, block_size=64), min_seconds)
    out["index_topk_prefill"] = {"value": reps * 32768 / dt, "unit": "queries/s", "cores": nthr, "kind": "port",
                                 "sample": f"the full 32,768 query rows (512 centroids, d=128, top-32) in fp32, "
                                           f"{reps} repeats in {dt:.1f} s; kernels/common.py ref_index_topk (torch)"}
    # gate superposition at the full [1,10,32768,64] shape
    o3 = [torch.randn(1, 10, 32768, 64, generator=g) for _ in range(3)]
    gz = torch.randn(1, 32768, 3, generator=g)
    reps, dt = _timed(lambda: C.ref_stream_superposition(o3[0], o3[1], o3[2], gate_logits=gz), min_seconds)
    out["stream_superposition"] = {"value": dt / reps * 1e6, "unit": "us/call", "cores": nthr, "kind": "port",
                                   "sample": f"the full shape in fp32, {reps} repeats in {dt:.1f} s; "
                                             f"kernels/common.py ref_stream_superposition (torch)"}
    return out


def decode_benches(dev, steps: int):
    import torch
    import torch.nn.functional as F
    from maba_sparse.kernels import hip_backend as hb
    out = {}
    # --- config 2b: 10,000 DGDA decode steps at B=64, H=10, d=64 (bf16 q/k/v, fp32 gates/state)
    B, H, d = 64, 10, 64
    g = torch.Generator().manual_seed(1)
    q = F.normalize(torch.randn(B, H, d, generator=g), dim=-1).to(dev, torch.bfloat16)
    k = F.normalize(torch.randn(B, H, d, generator=g), dim=-1).to(dev, torch.bfloat16)
    v = torch.randn(B, H, d, generator=g).to(dev, torch.bfloat16)
    la = (-F.softplus(torch.randn(B, H, 1, generator=g) + 2)).to(dev).expand(B, H, d)
    be = torch.sigmoid(torch.randn(B, H, 1, generator=g)).to(dev).expand(B, H, d)
    S = torch.zeros(B, H, d, d, device=dev)
    S2 = torch.zeros_like(S)
    o = torch.empty(B, H, d, device=dev)
    from maba_sparse import _native as N
    lib = N.load()
    dq, dk_, dv_, dla, db = N.desc(q), N.desc(k), N.desc(v), N.desc(la), N.desc(be)
    dS, dS2, do = N.desc(S), N.desc(S2), N.desc(o)
    def step():
        sp = N.stream_ptr(dev)   # the capture stream while a graph is recorded
        rc = lib.maba_hip_dgda_step(dq, dk_, dv_, None, dla, db, db, dS, do, dS2, sp)
        rc |= lib.maba_hip_dgda_step(dq, dk_, dv_, None, dla, db, db, dS2, do, dS, sp)
        if rc:
            N.check(rc, "dgda_step")

    def hundred_steps():
        for _ in range(50):
            step()
        return o

    # 10,000 state updates: a HIP graph of 100 launches replayed 100 times
    ms = graph_time(hundred_steps, 100, check=False)
    us = ms * 1e3 / 100
    eager_ms, _ = time_op(step, 500, 10)
    byts = 2 * B * H * d * d * 4 + B * H * (3 * d * 2 + 2 * 4 + d * 4)
    out["dgda_step_B64"] = {"us_per_step": us, "gbs": byts / (us * 1e-6) / 1e9, "steps": 10000,
                            "eager_us_per_step": eager_ms * 1e3 / 2, "algorithmic_bytes": byts}
    log(f"dgda_step B=64: {us:.2f} us/step")

    # --- configs 3/4: 1M-token latent cache, B=8, d_c=128
    B, L, dc, Hq, H, dh, K = 8, 1_000_000, 128, 10, 10, 64, 32
    gen = torch.Generator(device=dev).manual_seed(2)
    c_kv = torch.randn(B, L, dc, device=dev, generator=gen, dtype=torch.bfloat16)
    pos = torch.randint(0, L, (B,), generator=torch.Generator().manual_seed(3))
    for b in range(B):   # one salient token per sequence, norm x8
        c_kv[b, pos[b]] *= 8
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cent = hb.hip_compute_centroids(c_kv, block_size=64)
    hca = hb.hip_hca_pool(c_kv, pool=64)
    torch.cuda.synchronize()
    pool_ms, _ = time_op(lambda: hb.hip_compute_centroids(c_kv, block_size=64), 10, 2)
    out["centroid_pool_1M"] = {"us": pool_ms * 1e3, "gbs": B * L * dc * 2 / (pool_ms * 1e-3) / 1e9}
    log(f"centroid pooling 1M: {pool_ms * 1e3:.1f} us")
    q_idx = torch.randn(B, Hq, dc, device=dev, generator=gen, dtype=torch.bfloat16)
    q_lat = torch.randn(B, H, dc, device=dev, generator=gen) * 0.1
    gate = torch.randn(B, 3, device=dev, generator=gen)
    scale = 1.0 / math.sqrt(dh)
    nb = cent.shape[1]

    def indexer():
        return hb.hip_index_topk_decode(q_idx, cent, lambda_dist=0.1, top_k=K)     # [B, 10, 32] per head

    idx_fixed = indexer()

    def maba_sa():
        return hb.hip_maba_sa_decode(q_lat, c_kv, hca, idx_fixed, gate, L=L, scale=scale)

    def decode_step():
        return hb.hip_maba_sa_decode(q_lat, c_kv, hca, indexer(), gate, L=L, scale=scale)

    reps = max(steps * 10, 50)
    idx_ms = graph_time(indexer, reps)
    sa_ms = graph_time(maba_sa, reps)
    step_ms = graph_time(decode_step, reps)
    step_eager_ms, _ = time_op(decode_step, reps, 5)
    idx_eager_ms, _ = time_op(indexer, reps, 5)
    sa_eager_ms, _ = time_op(maba_sa, reps, 5)
    idx_bytes = B * nb * dc * 2
    nloc = 132
    sa_bytes = B * (hca.shape[1] * dc * 2 + H * K * 64 * dc * 2 + nloc * dc * 2)
    # us_per_step: the faster of graph replay and back-to-back eager calls (events around the
    # loop; the host enqueues ahead of the GPU, and the stream keeps steps from overlapping)
    idx_us, sa_us = min(idx_ms, idx_eager_ms) * 1e3, min(sa_ms, sa_eager_ms) * 1e3
    step_us = min(step_ms, step_eager_ms) * 1e3
    timing = "the faster of HIP graph replay and back-to-back eager calls, events on the stream"
    out["index_topk_decode_1M"] = {"us_per_step": idx_us, "gbs": idx_bytes / (idx_us * 1e-6) / 1e9,
                                   "graph_us_per_step": idx_ms * 1e3, "eager_us_per_step": idx_eager_ms * 1e3,
                                   "timing": timing}
    out["maba_sa_decode_1M"] = {"us_per_step": sa_us, "gbs": sa_bytes / (sa_us * 1e-6) / 1e9,
                                "graph_us_per_step": sa_ms * 1e3, "eager_us_per_step": sa_eager_ms * 1e3,
                                "index_sets": "per head [8,10,32]", "timing": timing}
    tot_bytes = sa_bytes + idx_bytes
    out["indexer_plus_maba_sa_1M"] = {"us_per_step": step_us, "gbs": tot_bytes / (step_us * 1e-6) / 1e9,
                                      "hbm_frac": tot_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                      "algorithmic_bytes": tot_bytes, "graph_us_per_step": step_ms * 1e3,
                                      "eager_us_per_step": step_eager_ms * 1e3,
                                      "traffic": measured_traffic("decode_bytes_per_step"),
                                      "traffic_source": TRAFFIC_SOURCE,
                                      "timing": timing + " (the two entry points per step)"}
    log(f"indexer decode 1M: graph {idx_ms * 1e3:.1f} us, eager {idx_eager_ms * 1e3:.1f} us")
    log(f"MABA-SA decode 1M: graph {sa_ms * 1e3:.1f} us, eager {sa_eager_ms * 1e3:.1f} us")
    log(f"indexer + MABA-SA decode step 1M: graph {step_ms * 1e3:.1f} us, eager {step_eager_ms * 1e3:.1f} us")
    del c_kv
    return out


def row_benches(dev, only=None):
    """Secondary lines for hot-path rows outside the headline: DGDA prefill with
    per-channel gates (the layer's gate layout, config-2 shape) and the causal prefill
    index_topk."""
    import torch
    import torch.nn.functional as F
    from maba_sparse.kernels import hip_backend as hb
    out = {}
    want = lambda name: only is None or name in only  # noqa: E731
    if want("dgda"):
        B, H, T, d = 4, 10, 32768, 64
        g = torch.Generator(device="cpu").manual_seed(5)
        q = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1).to(dev, torch.bfloat16)
        k = F.normalize(torch.randn(B, H, T, d, generator=g), dim=-1).to(dev, torch.bfloat16)
        v = torch.randn(B, H, T, d, generator=g).to(dev, torch.bfloat16)
        la = (-F.softplus(torch.randn(B, H, T, d, generator=g) + 2.0)).to(dev)
        beta = torch.sigmoid(torch.randn(B, H, T, d, generator=g)).to(dev)
        wg = torch.sigmoid(torch.randn(B, H, T, d, generator=g)).to(dev)

        def pc_step():
            return hb.hip_dgda_prefill(q, k, v, log_alpha=la, b=beta, w=wg, chunk_size=64, out_dtype=torch.bfloat16,
                                       state_dtype=torch.float32, allow_mixed_dtypes=True)

        ms, _ = time_op(pc_step, 3, 1)
        nbytes = B * H * T * (3 * d * 2 + 3 * d * 4 + d * 2) + B * H * d * d * 4
        del la, beta, wg
        # the headline kernel with slow decay (log alpha x 0.005, about 0.6% per token): segment
        # transitions never vanish, so the aggregate, map-chain and fix-up passes do full work
        sc = dgda_prefill_case(dev, B, H, T, d)
        sc["log_alpha"] = (sc["log_alpha"][..., :1] * 0.005).expand(B, H, T, d)   # still per token (stride 0)

        def slow_step():
            return hb.hip_dgda_prefill(**sc, chunk_size=64, out_dtype=torch.bfloat16, state_dtype=torch.float32,
                                       allow_mixed_dtypes=True)

        ms_slow, _ = time_op(slow_step, 5, 1)
        sb = prefill_bytes(B, H, T, d)
        out["dgda_prefill_slow_decay"] = {
            "ms_per_step": ms_slow, "tokens_per_s": B * T / (ms_slow * 1e-3), "gbs": sb / (ms_slow * 1e-3) / 1e9,
            "hbm_frac": sb / (ms_slow * 1e-3) / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": sb,
            "mfma_frac": prefill_flops(B, H, T, d) / (ms_slow * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
            "config": "BASELINE config 2 (B=4 H=10 T=32768 d=64, bf16 q/k/v, fp32 per-token gates) with the log "
                      "decay scaled by 0.005"}
        log(f"dgda_prefill slow decay: {ms_slow:.3f} ms/step")
        del sc
        out["dgda_prefill_per_channel_gates"] = {
            "ms_per_step": ms, "tokens_per_s": B * T / (ms * 1e-3), "gbs": nbytes / (ms * 1e-3) / 1e9,
            "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": nbytes,
            "config": "B=4 H=10 T=32768 d=64, bf16 q/k/v, fp32 [B,H,T,64] decay/erase/write gates, bf16 out"}
        log(f"dgda_prefill per-channel gates: {ms:.3f} ms/step")
        del q, k, v
    if want("prologue"):
        out.update(prologue_benches(dev))
    if want("topk"):
        # causal prefill index_topk: one sequence of 32,768 queries over 512 block centroids
        Bq, L, di, K = 1, 32768, 128, 32
        qi = torch.randn(Bq, L, di, device=dev, dtype=torch.bfloat16)
        cent = torch.randn(Bq, L // 64, di, device=dev, dtype=torch.bfloat16)

        def topk_prefill():
            return hb.hip_index_topk(qi, cent, lambda_dist=0.5, top_k=K, block_size=64)

        ms, _ = time_op(topk_prefill, 5, 1)
        # scoring flops: every query against the centroids of the blocks at or before its own
        fl = 2 * di * Bq * sum(min(t // 64 + 1, L // 64) for t in range(0, L, 64)) * 64
        out["index_topk_prefill"] = {"ms_per_call": ms, "queries_per_s": Bq * L / (ms * 1e-3),
                                     "roofline": {"bound": "mfma", "achieved": fl / (ms * 1e-3) / 1e12,
                                                  "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                                  "frac": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                                                  "algorithmic_flops": fl, "traffic": None},
                                     "config": "B=1 L=32768 d=128 bf16, 512 centroids, top-32, causal"}
        log(f"index_topk prefill 32k x 512: {ms:.3f} ms")
        del qi, cent
    if want("superposition"):
        # gate superposition of three prefill stream outputs [1, 10, 32768, 64] bf16 with
        # [1, 32768, 3] logits (the layer's prefill combine, sparse_attention.py:219)
        Bs, Hs, Ls, Ds = 1, 10, 32768, 64
        ol, os_, oh = (torch.randn(Bs, Hs, Ls, Ds, device=dev, dtype=torch.bfloat16) for _ in range(3))
        gl = torch.randn(Bs, Ls, 3, device=dev, dtype=torch.bfloat16)

        def superpose():
            return hb.hip_stream_superposition(ol, os_, oh, gate_logits=gl)

        ms, _ = time_op(superpose, 20, 3)
        sb = 4 * Bs * Hs * Ls * Ds * 2 + Bs * Ls * 3 * 2
        out["stream_superposition"] = {"us_per_call": ms * 1e3, "gbs": sb / (ms * 1e-3) / 1e9,
                                       "hbm_frac": sb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": sb,
                                       "config": "o_* [1,10,32768,64] bf16, gate logits [1,32768,3] bf16"}
        log(f"stream superposition 1x10x32768x64: {ms * 1e3:.1f} us")
        del ol, os_, oh, gl
    if want("prefill_attention"):
        out.update(prefill_attention_bench(dev))
    if want("layer_decode"):
        out["maba_sa_layer_decode_1M"] = layer_decode_bench(dev)
    if want("model"):
        out.update(model_decode_bench(dev))
    return out


def prefill_attention_bench(dev, B=1, H=10, L=32768, dh=64, dc=128, K=32):
    """MABA-SA prefill streams (local + sparse + HCA + gate) for a 32k-token sequence at the
    layer's default shape (10 heads of 64, d_c 128), each query's top-32 blocks from the HIP
    causal index_topk over random queries and centroids (lambda 0.5, the layer's default).

    Both fused forms of ``MabaSparseAttention`` are timed, as composites and as kernels: the
    latent form (``q_lat = W_k,h^T q_h``, one launch over the bf16 latent rows and their block
    means, ``o_h = W_v,h z_h``) and the head-space form (keys, values, block means and the
    early running means up-projected, one ``maba_sa_prefill`` launch).  ``ms_per_call`` and the
    roofline follow the form the layer picks for these selections (``_prefill_form``).  The
    roofline counts the reference's work: 4 d_head flops per key and head."""
    import torch
    from maba_sparse.kernels import hip_backend as hb
    from maba_sparse.layers.sparse_attention import PREFILL_UNION_LIMIT
    g = torch.Generator(device=dev).manual_seed(21)
    bf = lambda *sh: torch.randn(*sh, device=dev, generator=g, dtype=torch.bfloat16)  # noqa: E731
    q = bf(B, H, L, dh)
    c = bf(B, L, dc)
    Wk = torch.randn(H, dh, dc, device=dev, generator=g) * dc ** -0.5
    Wv = torch.randn(H, dh, dc, device=dev, generator=g) * dc ** -0.5
    gate = torch.randn(B, L, 3, device=dev, generator=g)
    idx = hb.hip_index_topk(bf(B, L, 64), bf(B, L // 64, 64), lambda_dist=0.5, top_k=K, block_size=64)
    grp = idx[:, : (L // 16) * 16].reshape(B, L // 16, 16 * K).sort(dim=-1).values
    distinct = (grp[..., 1:] != grp[..., :-1]).sum(dim=-1).float().mean().item() + 1.0
    form = "heads" if distinct < PREFILL_UNION_LIMIT * K else "latent"
    hca = hb.hip_hca_pool(c, pool=64)
    q_lat = torch.einsum("bhtd,hdc->bthc", q.float(), Wk).contiguous()
    z = torch.empty(B, L, H, dc, device=dev)

    def kernel_latent():
        return hb.hip_maba_sa_prefill_latent(q_lat, c, hca, idx, gate, scale=dh ** -0.5, out=z)

    def composite_latent():
        ql = torch.einsum("bhtd,hdc->bthc", q.float(), Wk).contiguous()
        means = hb.hip_hca_pool(c, pool=64)
        zz = hb.hip_maba_sa_prefill_latent(ql, c, means, idx, gate, scale=dh ** -0.5)
        return torch.einsum("bthc,hdc->bthd", zz, Wv)

    Wkb, Wvb = Wk.reshape(H * dh, dc).bfloat16(), Wv.reshape(H * dh, dc).bfloat16()
    heads = lambda t, n: t.view(B, n, H, dh).transpose(1, 2)  # noqa: E731
    cnt = torch.arange(1, 64, device=dev, dtype=torch.bfloat16).view(1, -1, 1)

    def head_inputs():   # as MabaSparseAttention._fused_prefill_heads forms them
        k, v = heads(c @ Wkb.t(), L), heads(c @ Wvb.t(), L)
        means = c.reshape(B, L // 64, 64, dc).mean(dim=2)
        kh, vh = heads(means @ Wkb.t(), L // 64), heads(means @ Wvb.t(), L // 64)
        early = heads((torch.cumsum(c[:, :63], dim=1) / cnt) @ Wvb.t(), 63)
        return k, v, kh, vh, early

    hin = head_inputs()

    def kernel_heads():
        return hb.hip_maba_sa_prefill(q, *hin, idx, gate, scale=dh ** -0.5)

    def composite_heads():
        return hb.hip_maba_sa_prefill(q, *head_inputs(), idx, gate, scale=dh ** -0.5)

    ms_l, _ = time_op(kernel_latent, 10, 2)
    ms_lc, _ = time_op(composite_latent, 10, 2)
    ms_h, _ = time_op(kernel_heads, 10, 2)
    ms_hc, _ = time_op(composite_heads, 10, 2)
    del hin
    ms, ms_comp = (ms_h, ms_hc) if form == "heads" else (ms_l, ms_lc)
    log(f"MABA-SA prefill 32k ({distinct / K:.2f} K distinct blocks per 16 queries, layer form {form}): "
        f"latent kernel {ms_l:.3f} ms (composite {ms_lc:.3f}), head-space kernel {ms_h:.3f} ms "
        f"(composite {ms_hc:.3f})")
    # keys per query: the local keys (window + sinks, fewer at the start), the listed blocks'
    # causal tokens and the complete means before the query
    pos = torch.arange(L, device=dev)
    n_loc = torch.clamp(pos + 1, max=128) + torch.clamp(torch.clamp(pos + 1 - 128, min=0), max=4)
    blk = idx[0].to(torch.int64)
    n_sp = torch.where(blk >= 0, torch.clamp(pos[:, None] - blk * 64 + 1, min=0, max=64), 0).sum(-1)
    n_hca = (pos + 1) // 64
    keys = (n_loc + n_sp + n_hca).double().sum().item()
    fl = keys * H * B * 4 * dh
    rf = {"bound": "mfma", "achieved": fl / (ms * 1e-3) / 1e12, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
          "frac": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, "algorithmic_flops": fl,
          "kernel": "maba_sa_prefill_kernel" if form == "heads" else "maba_sa_prefill_latent_kernel",
          "traffic": measured_traffic("maba_sa_prefill_heads_bytes_per_call" if form == "heads"
                                      else "maba_sa_prefill_latent_bytes_per_call"),
          "traffic_source": TRAFFIC_SOURCE}
    return {"maba_sa_prefill_32k": {
        "ms_per_call": ms_comp, "kernel_ms": ms, "form": form, "distinct_blocks_per_16_queries": distinct,
        "latent_kernel_ms": ms_l, "latent_composite_ms": ms_lc,
        "head_space_kernel_ms": ms_h, "head_space_composite_ms": ms_hc,
        "latent_form_flops": keys * H * B * 4 * dc,
        "queries_per_s": B * L / (ms_comp * 1e-3), "keys_per_query": keys / (B * L),
        "roofline": rf,
        "config": "B=1 H=10 d_head=64 d_c=128 L=32768 bf16, window 128 + 4 sinks, top-32 causal blocks per "
                  "query from index_topk (lambda 0.5), 512 HCA means; ms_per_call = the layer's form as a "
                  "composite (up-projections or q_lat / W_v projections, block means, kernel)"}}


def prologue_benches(dev, B=4, T=32768, dim=640, H=10):
    """The DGDA layer's prologue at the config-2 layer shape (bf16 projections -> bf16
    q/k/v and fp32 gates, the layer's HIP path), the same math as torch reference ops on
    the GPU, and the whole bf16 layer forward that uses it."""
    import torch
    from maba_sparse.kernels import common as C
    from maba_sparse.kernels import hip_backend as hb
    from maba_sparse.layers import DGDALayer
    out = {}
    Cc = 64 * H
    g = torch.Generator(device=dev).manual_seed(11)
    projs = torch.randn(B, T, 6 * Cc, device=dev, generator=g, dtype=torch.bfloat16).split(Cc, dim=-1)
    ws = [torch.randn(Cc, 1, 4, device=dev, generator=g) * 0.3 for _ in range(3)]
    hist = [torch.randn(B, Cc, 3, device=dev, generator=g, dtype=torch.bfloat16) for _ in range(3)]

    def fused():
        return hb.hip_dgda_prologue(projs, ws, hist, n_heads=H, gate_dtype=torch.float32, with_alpha=False)[0]

    def torch_ref():
        return C.ref_dgda_prologue(projs, ws, hist, n_heads=H, gate_dtype=torch.float32, with_alpha=False)[0]

    ms, _ = time_op(fused, 10, 2)
    ms_t, _ = time_op(torch_ref, 5, 1)
    nbytes = B * T * (6 * Cc * 2 + 3 * Cc * 2 + 3 * Cc * 4)
    out["dgda_layer_prologue"] = {
        "us_per_call": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "algorithmic_bytes": nbytes, "torch_reference_ops_us": ms_t * 1e3,
        "config": "B=4 T=32768 C=640 (10 heads x 64): six bf16 projections in, bf16 q/k/v + fp32 log_alpha/b/w out, "
                  "conv history carried"}
    log(f"dgda layer prologue: {ms * 1e3:.1f} us (torch reference ops {ms_t * 1e3:.1f} us)")
    del projs, ws, hist
    layer = DGDALayer(dim=dim, n_heads=H).to(dev, torch.bfloat16).eval()
    x = torch.randn(B, T, dim, device=dev, generator=g, dtype=torch.bfloat16)

    def fwd():
        with torch.no_grad():
            return layer(x)[0]

    ms, _ = time_op(fwd, 5, 1)
    layer.fuse_prologue = False
    ms_u, _ = time_op(fwd, 5, 1)
    layer.fuse_prologue = True
    # the fused prologue + recurrence passes alone, from the projections
    projs = torch.randn(B, T, 6 * Cc, device=dev, generator=g, dtype=torch.bfloat16).split(Cc, dim=-1)
    convs = (layer.conv_q.weight, layer.conv_k.weight, layer.conv_v.weight)
    ob = torch.empty(B, T, Cc, device=dev, dtype=torch.bfloat16)
    def fused_passes():
        with torch.no_grad():
            return hb.hip_dgda_layer_prefill(projs, convs, None, out=ob)

    ms_k, _ = time_op(fused_passes, 5, 1)
    out["dgda_layer_forward"] = {
        "ms_per_call": ms, "tokens_per_s": B * T / (ms * 1e-3), "unfused_ms_per_call": ms_u,
        "fused_prefill_ms": ms_k,
        "config": "DGDALayer(dim=640, 10 heads) bf16, x [4, 32768, 640], no_grad: one 640x3840 projection GEMM, "
                  "the per-channel-gate DGDA prefill with the prologue fused into its staging "
                  "(fused_prefill_ms: those passes alone), o_proj; unfused: the one-pass prologue kernel, "
                  "then the prefill on its stored outputs"}
    log(f"dgda layer forward (bf16, B=4, T=32768): {ms:.3f} ms fused, {ms_u:.3f} ms unfused; "
        f"fused prefill passes {ms_k:.3f} ms")
    return out


def model_decode_bench(dev, B=16, L=131072, steps=256):
    """the 101M Maba v2 stack (20 layers, 15 DGDA + 5 MABA-SA) in bf16 with
    N(0, 0.02) random weights, a prefill of B x L uniform random token ids, then greedy decode
    (one token from the prefill logits, steps - 1 single-token steps over the decode caches)."""
    import torch
    from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
    torch.manual_seed(0)
    model = MabaSparseForCausalLM(get_101m_config()).init_normal(0.02).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, model.config.vocab_size, (B, L), device=dev)
    marks = []

    def mark():
        torch.cuda.synchronize()
        marks.append(time.perf_counter())

    graph = model.serving_graph_ok(ids)
    # a short generation first: code objects, library handles and the allocator's pools are
    # set up there, not inside the timed prefill
    model.generate_greedy(ids[:, :2048], 4)
    mark()
    toks = model.generate_greedy(ids, steps, on_prefill_done=mark, on_graph_ready=mark)
    mark()
    prefill_s = marks[1] - marks[0]
    # the first decode step runs eagerly (library set-up) and the graph is then captured once;
    # ms_per_token times the steps replayed from the graph, decode_incl_setup_ms_per_token the
    # whole decode phase (eager first step and capture included) over every decode step
    if graph and len(marks) == 4:
        per_step = (marks[3] - marks[2]) / max(steps - 2, 1)
        whole = (marks[3] - marks[1]) / max(steps - 1, 1)
    else:
        per_step = whole = (marks[-1] - marks[1]) / max(steps - 1, 1)
    log(f"model config 5: prefill {prefill_s:.2f} s ({B * L / prefill_s / 1e6:.2f} M tok/s), decode "
        f"{per_step * 1e3:.2f} ms/step ({B / per_step:.0f} tok/s), graph={graph}")
    eager_steps = 17
    marks.clear()
    mark()
    model.generate_greedy(ids, eager_steps, on_prefill_done=mark, graph=False)
    mark()
    eager_step = (marks[2] - marks[1]) / (eager_steps - 1)
    log(f"model config 5, eager LatentCache loop: {eager_step * 1e3:.2f} ms/step")
    # algorithmic bytes of one decode step: every weight once (the tied embedding matrix once, as
    # the LM head), the DGDA states read and written, and per MABA-SA block its centroids, HCA
    # means, selected blocks and local window at the final context
    c = model.config
    n_params = sum(p.numel() for p in model.parameters())
    n_dgda = sum(1 for b in model.layers if not b.is_attention)
    n_sa = len(model.layers) - n_dgda
    Lf = L + steps
    state = 2 * B * c.n_heads * c.d_head * c.d_head * 2
    sa = B * ((Lf // 64) * c.d_idx * 2 + (Lf // 64) * c.d_c * 2 + c.top_k * 64 * c.d_c * 2 + 132 * c.d_c * 2)
    step_bytes = n_params * 2 + n_dgda * state + n_sa * sa
    out = {"model_decode_config5": {
        "ms_per_token": per_step * 1e3, "tokens_per_s": B / per_step, "decode_steps": steps - 1,
        "decode_incl_setup_ms_per_token": whole * 1e3,
        "serving_path": "one captured HIP graph per decode step" if graph else "eager",
        "eager_ms_per_token": eager_step * 1e3,
        "prefill_s": prefill_s, "prefill_tokens_per_s": B * L / prefill_s, "first_tokens": toks[0, :4].tolist(),
        "roofline": {"bound": "hbm", "achieved": step_bytes / per_step / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": step_bytes / per_step / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": step_bytes,
                     "traffic": None},
        "config": f"101M Maba v2 (20 layers, 3:1 DGDA:MABA-SA, d_model 640, factorised 32768->128->640 "
                  f"embedding, SwiGLU 1248, RMSNorm), bf16 weights ~N(0,0.02), B={B}, prefill {L} uniform "
                  f"random ids, {steps} greedy tokens (one from the prefill, {steps - 1} decode steps)"}}
    del model, ids
    torch.cuda.empty_cache()
    return out


def layer_decode_bench(dev, B=8, L0=1_000_000 - 10, steps=20):
    """The MABA-SA layer's decode step (layers/sparse_attention.py:221-277 orchestration):
    latent append, indexer (projections, key/centroid cache, decode top-32), the fused
    streams and the head projections, eager, at a 1M-token context held in synthetic
    caches (B=8, d_model 640, 10 heads of 64, d_c 128, d_idx 64, bf16)."""
    import torch
    from maba_sparse.kernels import hip_backend as hb
    from maba_sparse.layers.sparse_attention import LatentCache, MabaSparseAttention
    from maba_sparse.layers.indexer import _Growing
    torch.manual_seed(11)
    layer = MabaSparseAttention(dim=640, n_heads=10, d_head=64, d_c=128, window_size=128, block_size=64,
                                top_k=32, hca_pool_size=64, dist_lambda=0.1, d_idx=64)
    layer = layer.to(dev, torch.bfloat16).eval()
    cap = L0 + steps + 16
    cache = LatentCache(B, cap, 128, pool=64, device=dev, dtype=torch.bfloat16)
    cache.c[:, :L0].normal_()
    cache.n = L0
    full = L0 // 64
    cache.hca[:, :full] = hb.hip_hca_pool(cache.c[:, : full * 64], pool=64)
    cache.nh = full
    keys = torch.randn(B, L0, 64, device=dev, dtype=torch.bfloat16)
    layer.indexer._keys = _Growing(keys)
    layer.indexer._cents = _Growing(hb.hip_compute_centroids(keys[:, : full * 64], block_size=64))
    del keys
    x = torch.randn(B, 1, 640, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        for _ in range(3):
            layer.decode_step(x, cache)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            layer.decode_step(x, cache)
        e1.record()
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    nb = cache.n // 64
    byts = B * (nb * 64 * 2 + nb * 128 * 2 + 32 * 64 * 128 * 2 + 132 * 128 * 2)   # centroids, HCA, sparse, local
    log(f"MABA-SA layer decode step at 1M (eager): {us:.1f} us")
    # the serving path: DeviceCache appends and device-length kernels, one captured graph per step
    from maba_sparse.layers.sparse_attention import DeviceCache
    n0 = cache.n
    dcache = DeviceCache(cache.c[:, :n0], layer.indexer._keys.view()[:, :n0], n0 + 2 * steps + 8)
    del cache
    counters = torch.tensor([n0, n0 + 1], dtype=torch.long, device=dev)
    with torch.no_grad():
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            layer.decode_step_device(x, dcache, counters)
            counters += 1
        torch.cuda.current_stream(dev).wait_stream(side)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            layer.decode_step_device(x, dcache, counters)
            counters += 1
        for _ in range(3):
            gr.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
    gus = e0.elapsed_time(e1) / steps * 1e3
    log(f"MABA-SA layer decode step at 1M (device-resident, graph replay): {gus:.1f} us")
    del dcache, layer
    return {"us_per_step": gus, "gbs": byts / (gus * 1e-6) / 1e9, "hbm_frac": byts / (gus * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "algorithmic_bytes": byts, "steps": steps, "eager_us_per_step": us,
            "timing": "one captured HIP graph per step (cache append, decode indexer, fused streams, projections), "
                      "events around back-to-back replays; eager_us_per_step: the LatentCache decode_step",
            "config": "B=8, context ~1M (synthetic latent, key and centroid caches), d_model 640, 10 heads x 64, "
                      "d_c 128, d_idx 64, one indexer query shared by the heads, top-32, bf16"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); multi-GPU sharding is "
              f"designed (per-GPU shards of (b, h) pairs, indexer blocks and decode segments) but not launched",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from maba_sparse.kernels import hip_backend as hb
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)     # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "copies": 5}), flush=True)
        return
    if args.only_decode:
        print(json.dumps({"decode": decode_benches(dev, args.steps)}), flush=True)
        return
    if args.only_rows:
        print(json.dumps({"rows": row_benches(dev, args.row.split(",") if args.row else None)}), flush=True)
        return
    if args.only_model:
        print(json.dumps({"rows": model_decode_bench(dev, args.model_batch, args.model_prefill, args.model_steps)}),
              flush=True)
        return
    B, H, T, d = 4, 10, 32768, 64
    inp = dgda_prefill_case(dev, B, H, T, d)
    log("dgda_prefill config 2 inputs ready")

    def step():
        return hb.hip_dgda_prefill(**inp, chunk_size=64, out_dtype=torch.bfloat16, state_dtype=torch.float32,
                                   allow_mixed_dtypes=True)

    ms, wall_ms = time_op(step, args.steps, args.warmup)
    log(f"dgda_prefill: {ms:.3f} ms/step (wall {wall_ms:.3f})")
    tok_s = B * T / (ms * 1e-3)
    nbytes = prefill_bytes(B, H, T, d)
    flops = prefill_flops(B, H, T, d)
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = measured_traffic("dgda_prefill_bytes_per_step")
    res = {
        "metric": "DGDA prefill tok/s @T=32k; MABA-SA decode us/step @1M ctx; % roofline",
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded BASELINE config 2 distributions)",
        "config": {"workload": "dgda_prefill BASELINE config 2", "batch": B, "heads": H, "seq_len": T,
                   "d_k": d, "d_v": d, "chunk": 64, "qkv": "bf16", "gates": "fp32 per-token (stride-0)",
                   "state": "fp32", "out": "bf16", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "dgda_prefill op (aggregate + zero-start + fix-up launches)",
                     "algorithmic_bytes": nbytes},
        "mfma": {"achieved": flops / (ms * 1e-3) / 1e12, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, "algorithmic_flops": flops},
    }
    if not args.only_prefill and not args.skip_decode:
        res["decode"] = decode_benches(dev, args.steps)
        res["rows"] = row_benches(dev)
    if not args.only_prefill and not args.skip_cpu:
        log("timing the CPU baseline")
        res["cpu_baseline"] = cpu_baseline()
        log("timing the config-1 CPU anchor")
        res["cpu_anchor_config1"] = cpu_anchor_config1()
        if not args.skip_decode:
            log("timing the CPU baselines of the secondary rows")
            rows_cpu = cpu_row_baselines()
            for name, cb in rows_cpu.items():
                for section in ("decode", "rows"):
                    if name in res.get(section, {}):
                        res[section][name]["cpu_baseline"] = cb
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
