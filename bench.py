"""Benchmark of the batch-invariant GEMM + SDPA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the GEMM sweep, at M = 256 where the
roofline target applies): one step = bi.matmul over the five (K, N) shapes of
the sweep, (256, K) bf16 activations ~ N(0, 1) times (K, N) bf16 weights
~ N(0, 1/K), seeded. `value` is the step's total flops / wall time, inputs
resident in HBM. Alongside, on the same run:
  * roofline of the dominant kernel (256 x 4096 x 32000), its average
    duration over every other timed step from HIP events that the launch
    itself records (the kernel's own start and end timestamps);
  * stock torch.matmul (hipBLASLt) on the same inputs, interleaved;
  * the same sweep in f16 and fp32 (fp32 against the 157.3 TFLOP/s fp32
    MFMA peak);
  * a sustained leg: the same step repeated for --sustained seconds, its
    dominant launch self-timed in every 16th step (roofline.sustained);
  * decode SDPA (configs[2]: B = 64, 32/8 heads, D = 128, N = 8192) GB/s, a
    decode sweep over B in {1, 8, 64} x N in {2048, 8192} (eager calls, against
    stock), and graph-timed cells B in {1, 2, 4, 8} x N in {2048, 8192} (20
    calls replayed as one HIP graph: device time, where eager calls of these
    sizes are bound by the host's per-call cost);
  * causal prefill SDPA (B = 1, 32/8 heads, D = 128, 2048 x 2048) TFLOP/s,
    against stock torch SDPA;
  * the configs[4] prefill GEMMs at M = 4096 (bi.linear on (N, K) weights,
    against stock F.linear, each launch timed inside the steps) against the
    MFMA peak, and the feed probe (bi_feed_probe: the GEMM ring's operand
    stream with no arithmetic, from L2 and from HBM);
  * 4-bit affine quantized linear (4096 x 4096, group 64) at M = 1 and 256,
    against stock dequantize + F.linear;
  * a bit-invariance check of row 0 of every shape across batch sizes 1..256;
  * the configs[4] decoder's prefill at batch 8 and the bits of sequence 0's
    logits against batch 1, invariant and stock (--no-model skips it);
  * the CPU baseline on the host cores this process may use: the oracle's
    fixed-order fp32 restatements of the reference GEMM and attention (C,
    OpenMP) on bounded samples of the same workloads, beside stock torch.
Every GPU entry carries its roofline fraction: achieved / min(MFMA peak,
arithmetic intensity x HBM peak) for the GEMMs and prefill attention, and
achieved / HBM peak for decode attention and the quantized linear.
Prints one JSON line.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "mlx-batch-invariant_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "bi-GEMM TFLOP/s & SDPA GB/s vs roofline; 0 bits differ across batch 1-256"
M = 256
SHAPES = [(512, 512), (4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]  # (K, N)
DOMINANT = (4096, 32000)
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}  # dense MFMA peaks
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SDPA = dict(B=64, H=32, Hkv=8, N=8192, D=128)
CPU_ROWS = 256              # rows of M per shape in the CPU sample (all of them)
CPU_SECONDS = 10.0          # repeat whole passes until at least this long
CPU_SDPA_B = 4              # batch entries of configs[2] in the CPU attention sample
CPU_SDPA_SECONDS = 5.0
SUSTAINED_S = 1.5           # seconds of repeated steps in the sustained leg
PREFILL_M = 4096            # rows of the configs[4] prefill GEMMs (batch 8 x 512 tokens)


def gemm_flops(m, k, n):
    return 2.0 * m * k * n


def gemm_bytes(m, k, n, esize=2):
    return float(m * k + k * n + m * n) * esize


def sdpa_bytes(B, H, Hkv, N, D, esize=2):
    return float(2 * B * Hkv * N * D + 2 * B * H * 1 * D) * esize


def make_inputs(torch, dev, dtype=None, seed=0):
    dtype = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    ops = []
    for K, N in SHAPES:
        a = torch.randn(M, K, generator=g).to(dtype)
        w = (torch.randn(K, N, generator=g) / math.sqrt(K)).to(dtype)
        ops.append((a, w, a.to(dev), w.to(dev)))
    return ops


def gemm_roof(m, k, n, us, dname="bf16"):
    """Roofline figures of one GEMM launch of `us` microseconds."""
    es = 4 if dname == "f32" else 2
    fl, by = gemm_flops(m, k, n), gemm_bytes(m, k, n, es)
    tf = fl / us / 1e6
    roof = min(PEAK_TFLOPS[dname], fl / by * PEAK_HBM_GBS / 1e3)
    return {"tflops": round(tf, 1), "gbps": round(by / us / 1e3, 1),
            "frac_of_min_roof": round(tf / roof, 4),
            "mfma_frac": round(tf / PEAK_TFLOPS[dname], 4),
            "hbm_frac": round(by / us / 1e3 / PEAK_HBM_GBS, 4),
            "bound": "hbm" if roof < PEAK_TFLOPS[dname] else "mfma"}


def host_cores():
    """(cores this process may use, cores visible): the affinity mask, capped by
    the cgroup CPU quota where one is set (a GPU box's share of a larger host)."""
    vis = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(per)))
    except (OSError, ValueError):
        pass
    return (min(vis, quota) if quota else vis), vis


def load_traffic():
    """HBM bytes per launch of the dominant kernel, measured with rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE and scaled by a copy-kernel calibration; the
    summary is committed under profiles/. None when absent."""
    path = os.path.join(REPO, "profiles", "gemm_bf16_256x4096x32000_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(ops):
    """Oracle fixed-order fp32 GEMM (C, OpenMP, every core this process may
    use) on the first CPU_ROWS rows of every shape of the step; the oracle's
    fixed-order attention on CPU_SDPA_B batch entries of configs[2]; stock
    torch on the same samples."""
    cores, visible = host_cores()
    os.environ["OMP_NUM_THREADS"] = str(cores)
    import numpy as np

    from oracle import gemm as ogemm

    lib = ogemm.clib()
    prepared = []
    for a, w, _, _ in ops:
        a32 = np.ascontiguousarray(a[:CPU_ROWS].float().numpy())
        bt = np.ascontiguousarray(w.float().numpy().T)  # (N, K): contiguous inner loop
        prepared.append((a32, bt, np.empty((CPU_ROWS, bt.shape[0]), dtype=np.float32)))
    flops, passes = 0.0, 0
    t0 = time.perf_counter()
    while passes == 0 or time.perf_counter() - t0 < CPU_SECONDS:
        for a32, bt, out in prepared:
            lib.oracle_gemm_bt(ogemm.fptr(a32), ogemm.fptr(bt), ogemm.fptr(out), CPU_ROWS,
                               bt.shape[0], a32.shape[1])
            flops += gemm_flops(CPU_ROWS, a32.shape[1], bt.shape[0])
        passes += 1
    dt = time.perf_counter() - t0

    # Beside it: stock torch on the CPU (fp32 matmul, same rows and shapes) and
    # the reference's own CPU backend, MLX, when it is importable.
    import importlib.util

    import torch

    torch.set_num_threads(cores)
    tt = [(torch.from_numpy(a32), torch.from_numpy(bt).t()) for a32, bt, _ in prepared]
    tflops, tpasses = 0.0, 0
    t1 = time.perf_counter()
    while tpasses == 0 or time.perf_counter() - t1 < 2.0:
        for a32, b32 in tt:
            torch.matmul(a32, b32)
            tflops += gemm_flops(CPU_ROWS, a32.shape[1], b32.shape[1])
        tpasses += 1
    tdt = time.perf_counter() - t1
    sdpa = cpu_sdpa_baseline(torch, np)
    mlx = importlib.util.find_spec("mlx") is not None
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": cores,
            "cores_visible": visible,
            "kind": "port",
            "sample": "%d pass(es) over the first %d of the %d rows of each of the 5 (K,N) "
                      "shapes; fixed-order fp32 fmaf restatement of the reference K loop "
                      "(oracle/csrc/oracle.c), %.1f s on %d threads" % (passes, CPU_ROWS, M, dt,
                                                                         cores),
            "torch_cpu_tflops": round(tflops / tdt / 1e12, 4),
            "sdpa": sdpa,
            "mlx_cpu": ("mlx is importable but its CPU timing is not built in this bench"
                        if mlx else "unavailable: mlx is not installed on this host")}


def cpu_sdpa_baseline(torch, np):
    """configs[2] decode attention on the host: the oracle's fixed-order fp32
    restatement of the reference kernel (32 key-stride partials, C, OpenMP over
    batch x head x row) and stock torch CPU SDPA, on CPU_SDPA_B of the 64 batch
    entries, reported as the algorithmic bytes of the sample per second."""
    from oracle import sdpa as osdpa

    B, H, Hkv, N, D = CPU_SDPA_B, SDPA["H"], SDPA["Hkv"], SDPA["N"], SDPA["D"]
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).float().numpy()
    k = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16).float().numpy()
    v = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16).float().numpy()
    by = sdpa_bytes(B, H, Hkv, N, D)
    passes, t0 = 0, time.perf_counter()
    while passes == 0 or time.perf_counter() - t0 < CPU_SDPA_SECONDS:
        osdpa.sdpa_fixed32(q, k, v, scale=1.0 / math.sqrt(D))
        passes += 1
    dt = time.perf_counter() - t0
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    tpasses, t1 = 0, time.perf_counter()
    while tpasses == 0 or time.perf_counter() - t1 < 2.0:
        torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, enable_gqa=True)
        tpasses += 1
    tdt = time.perf_counter() - t1
    return {"value": round(by * passes / dt / 1e9, 3), "unit": "GB/s",
            "sample": "%d pass(es) over %d of the 64 batch entries of configs[2] (32/8 heads, "
                      "D=128, N=8192, qL=1), bytes counted as bf16 like the GPU figure; "
                      "fixed-order fp32 restatement of the reference attention "
                      "(oracle/csrc/oracle.c), %.1f s" % (passes, B, dt),
            "torch_cpu_gbps": round(by * tpasses / tdt / 1e9, 3)}


def progress(leg):
    """One stderr line as each leg starts (the JSON line stays alone on stdout)."""
    print("bench.py: %s" % leg, file=sys.stderr, flush=True)


def graph_us(torch, fn, calls=20, replays=7):
    """Device time of one fn() call: `calls` calls captured in a HIP graph,
    replayed `replays` times between HIP events; median replay / calls."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / calls)
    del graph
    return statistics.median(times)


def feed_probe(torch, dev, reps=10):
    """The per-CU operand feed that bounds the large-M GEMM (bi_feed_probe):
    256 workgroups, one per CU, each stream 8 MB in 32 KB stages through the
    256 x 256 footprints' LDS ring with no arithmetic, from one shared 2 MiB
    panel (L2-resident after the first pass) and from 256 distinct 4 MiB
    panels (HBM). A 256 x 256 tile consumes 32 KB per chunk-step of
    2 * 256 * 256 * 32 flop, 31.8 B/clk per CU at the dense bf16 peak (4069
    flop/clk per CU at 2.4 GHz), so feed / 31.8 bounds its MFMA fraction."""
    from mlx_batch_invariant import _lib

    L = _lib.lib()
    buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    stages, wgs = 256, 256
    need = 32768 / (2.0 * 256 * 256 * 32 / (PEAK_BF16_TFLOPS * 1e12 / (256 * 2.4e9)))
    out = {"bytes_per_clk_per_cu_needed_256x256": round(need, 1)}
    for name, panel, panels in (("l2_shared_2MiB", 2 << 20, 1), ("hbm_256x4MiB", 4 << 20, 256)):
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()  # creates the HIP events
            e1.record()
            torch.cuda.synchronize()
            _lib.check(L.bi_feed_probe(buf.data_ptr(), panel, panels, stages, wgs, e0.cuda_event,
                                       e1.cuda_event, torch.cuda.current_stream().cuda_stream),
                       "bi_feed_probe")
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        us = statistics.median(ts)
        byts = float(wgs) * stages * 32768
        bpc = byts / wgs / (us * 1e-6 * 2.4e9)
        out[name] = {"us": round(us, 2), "gbps": round(byts / us / 1e3, 1),
                     "bytes_per_clk_per_cu": round(bpc, 2),
                     "mfma_frac_bound_256x256": round(bpc / need, 3)}
    del buf
    torch.cuda.empty_cache()
    return out


def prefill_gemms(torch, bi, dev, steps=8, warmup=3):
    """configs[4]'s prefill GEMMs at batch 8 x 512 tokens (M = 4096 rows),
    bi.linear on (N, K) weights, bf16: one step runs the four (K, N) shapes of
    the sweep in turn (474 MB of weights, more than the Infinity Cache), each
    bi launch timed by its own timestamps and each stock F.linear (hipBLASLt)
    by HIP events, inside the steps. MFMA-bound: fractions of the 2.5 PFLOP/s
    dense bf16 peak."""
    from mlx_batch_invariant import _gemm

    g = torch.Generator().manual_seed(5)
    Mp = PREFILL_M
    ops = []
    for K, N in SHAPES[1:]:
        x = torch.randn(Mp, K, generator=g).to(torch.bfloat16).to(dev)
        w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
        ops.append((K, N, x, w))
    ev = lambda: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    bi_ev = [[ev() for _ in ops] for _ in range(steps)]
    st_ev = [[ev() for _ in ops] for _ in range(steps)]
    for row in bi_ev + st_ev:
        for e0, e1 in row:
            e0.record()
            e1.record()
    torch.cuda.synchronize()
    for s_ in range(warmup + steps):
        for i, (K, N, x, w) in enumerate(ops):
            if s_ >= warmup:
                _gemm.linear_timed(x, w, *bi_ev[s_ - warmup][i])
            else:
                bi.linear(x, w)
        for i, (K, N, x, w) in enumerate(ops):
            if s_ >= warmup:
                e0, e1 = st_ev[s_ - warmup][i]
                e0.record()
                torch.nn.functional.linear(x, w)
                e1.record()
            else:
                torch.nn.functional.linear(x, w)
    torch.cuda.synchronize()
    shapes, tot_fl, tot_bi, tot_st = [], 0.0, 0.0, 0.0
    for i, (K, N, x, w) in enumerate(ops):
        tb = statistics.median(bi_ev[s_][i][0].elapsed_time(bi_ev[s_][i][1]) * 1e3
                               for s_ in range(steps))
        ts = statistics.median(st_ev[s_][i][0].elapsed_time(st_ev[s_][i][1]) * 1e3
                               for s_ in range(steps))
        fl = gemm_flops(Mp, K, N)
        tot_fl, tot_bi, tot_st = tot_fl + fl, tot_bi + tb, tot_st + ts
        shapes.append({"M": Mp, "K": K, "N": N, "bi_us": round(tb, 1),
                       "bi_tflops": round(fl / tb / 1e6, 1),
                       "mfma_frac": round(fl / tb / 1e6 / PEAK_BF16_TFLOPS, 4),
                       "stock_us": round(ts, 1), "stock_tflops": round(fl / ts / 1e6, 1),
                       "stock_mfma_frac": round(fl / ts / 1e6 / PEAK_BF16_TFLOPS, 4),
                       "geometry": _gemm.geometries()[
                           _gemm._lib.lib().bi_gemm_pick_geometry(Mp, N, K, 2, 1)]})
    del ops
    torch.cuda.empty_cache()
    return {"config": "configs[4] prefill GEMMs: M=%d (batch 8 x 512 tokens), bi.linear (N,K) "
                      "weights, bf16, the four (K,N) shapes of the sweep per step" % Mp,
            "steps_timed": steps, "shapes": shapes,
            "bi_tflops": round(tot_fl / tot_bi / 1e6, 1),
            "mfma_frac": round(tot_fl / tot_bi / 1e6 / PEAK_BF16_TFLOPS, 4),
            "stock_tflops": round(tot_fl / tot_st / 1e6, 1),
            "stock_mfma_frac": round(tot_fl / tot_st / 1e6 / PEAK_BF16_TFLOPS, 4)}


def model_determinism(torch, bi, dev):
    """random-init 32-layer Llama-shaped decoder, 512-token seeded
    prompt; bits of sequence 0's last-position logits at batch 8 vs batch 1,
    under batch_invariant_mode and stock; and the prefill time of both paths
    at batch 8 (HIP events, median of 3)."""
    from mlx_batch_invariant import decoder

    m = decoder.build(decoder.LLAMA_7B_SHAPE, device=dev, seed=0)
    ids = decoder.prompts(m.c, 8, 512, seed=0, device=dev)
    out = {"config": "configs[4]: %d layers, hidden %d, %d/%d heads, FFN %d, vocab %d, bf16, "
                     "512-token prompt; sequence 0 at batch 8 vs batch 1"
                     % (m.c.layers, m.c.hidden, m.c.heads, m.c.kv_heads, m.c.inter, m.c.vocab)}
    for label, inv in (("invariant", True), ("stock", False)):
        base = decoder.logits_bits(m, ids[:1], inv)
        out["%s_bits_differing" % label] = int((decoder.logits_bits(m, ids, inv) != base).sum())
        times = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            decoder.logits_bits(m, ids, inv)
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        out["%s_prefill_ms_batch8" % label] = round(statistics.median(times), 2)
    out["logits"] = m.c.vocab
    del m
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the 32-layer decoder determinism check (configs[4])")
    ap.add_argument("--sustained", type=float, default=SUSTAINED_S, metavar="SECONDS",
                    help="length of the sustained leg (default %(default)s s; 0: as many steps "
                         "as the burst, e.g. for counter passes, where every dispatch is "
                         "serialised with its counter readout)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy three times (the known-size "
                         "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--feed-probe", action="store_true",
                    help="only run the per-CU operand feed probe (bi_feed_probe) and print it")
    ap.add_argument("--quantized", action="store_true",
                    help="only run the 4-bit quantized linear (4096x4096, group 64) and the "
                         "dense bi.linear on the same shape, at 1 and 256 rows, five launches "
                         "each (for counter passes)")
    ap.add_argument("--prefill-gemm", action="store_true",
                    help="only run the four configs[4] prefill GEMMs at M=4096 (bi.linear, "
                         "(N, K) weights, bf16), six launches each, each followed by a "
                         "synchronisation (for counter passes)")
    ap.add_argument("--prefill-shape", choices=("rows", "shared"),
                    help="only run the causal prefill (B=1, 32/8 heads, L=2048, D=128, bf16) "
                         "five times through one forced attention launch shape (for counter "
                         "passes of one kernel)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the invariant GEMM and attention have no "
              "multi-GPU path in this build (--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch

    import mlx_batch_invariant as bi
    from mlx_batch_invariant import _gemm

    def bits(t):  # raw bit pattern of a 16-bit float tensor
        return t.detach().contiguous().view(torch.int16).cpu()

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes": src.numel() * 4}))
        return
    if args.feed_probe:
        print(json.dumps({"feed_probe": feed_probe(torch, dev)}))
        return
    if args.quantized:
        g = torch.Generator().manual_seed(0)
        wq = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16)
        qw, qs, qz = (t.to(dev) for t in bi.quantize(wq, 64, 4))
        wd = wq.to(dev)
        for Mq in (1, 256):
            xq = torch.randn(Mq, 4096, generator=g).to(torch.bfloat16).to(dev)
            for _ in range(5):
                bi.quantized_linear(xq, qw, qs, qz, 64, 4)
            for _ in range(5):
                bi.linear(xq, wd)
        torch.cuda.synchronize()
        print(json.dumps({"quantized": "4-bit g64 4096x4096 and dense bf16, M in (1, 256)",
                          "launches": 5}))
        return
    if args.prefill_gemm:
        g = torch.Generator().manual_seed(0)
        for K, N in ((4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)):
            xg = torch.randn(4096, K, generator=g).to(torch.bfloat16).to(dev)
            wg = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16).to(dev)
            for _ in range(6):
                bi.linear(xg, wg)
                torch.cuda.synchronize()
            del xg, wg
        print(json.dumps({"prefill_gemm": "M=4096 bi.linear on (K, N) in (4096, 4096), "
                          "(4096, 11008), (11008, 4096), (4096, 32000)", "launches": 6}))
        return
    if args.prefill_shape:
        from mlx_batch_invariant import _attention, _lib
        shape = {"rows": _lib.SDPA_ROWS, "shared": _lib.SDPA_SHARED}[args.prefill_shape]
        g = torch.Generator().manual_seed(0)
        L, D = 2048, SDPA["D"]
        q, k, v = (torch.randn(1, h, L, D, generator=g).to(torch.bfloat16).to(dev)
                   for h in (SDPA["H"], SDPA["Hkv"], SDPA["Hkv"]))
        for _ in range(5):
            _attention._sdpa_eager(q, k, v, 1.0 / math.sqrt(D), _lib.MASK_CAUSAL, None,
                                   (0, 0, 0), 0, None, shape)
        torch.cuda.synchronize()
        print(json.dumps({"prefill_shape": args.prefill_shape, "launches": 5}))
        return
    ops = make_inputs(torch, dev)
    step_flops = sum(gemm_flops(M, K, N) for K, N in SHAPES)
    dom = SHAPES.index(DOMINANT)

    def step(outs=None):
        for i, (_, _, a, w) in enumerate(ops):
            y = bi.matmul(a, w)
            if outs is not None:
                outs.append(y)

    progress("steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: exactly --steps steps, synchronised on both sides. In
    # every other step (every step when there are fewer than four) the
    # dominant kernel's launch records its own start and end timestamps into
    # a pair of HIP events (bi_gemm_timed, same kernel and arguments as
    # bi.matmul): event markers between the launches would idle the GPU for
    # several microseconds each and be counted in the kernel's time. The
    # self-timed launch in every step cost about 3 us of a 200 us step, in
    # every other step about 1 us; single launches vary by a few per cent,
    # so fewer samples made the average noisy.
    timed = range(1, args.steps, 2) if args.steps >= 4 else range(args.steps)
    evs = {s: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for s in timed}
    for e0, e1 in evs.values():  # torch creates the underlying HIP event on its first record
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for i, (_, _, a, w) in enumerate(ops):
            if i == dom and s in evs:
                _gemm.matmul_timed(a, w, *evs[s])
            else:
                bi.matmul(a, w)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = step_flops * args.steps / elapsed / 1e12
    dom_us = statistics.mean(e0.elapsed_time(e1) for e0, e1 in evs.values()) * 1e3

    progress("sustained")
    # Sustained: the same step repeated for at least --sustained seconds (the
    # burst above covers a few milliseconds; the dominant kernel slows by
    # several per cent under longer load), the dominant launch self-timed in
    # every 16th step.
    n_sus = max(args.steps, int(math.ceil(args.sustained * 1e3 / ms_per_step)))
    sus_timed = list(range(min(8, n_sus // 2), n_sus, 16))
    sus_evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in sus_timed]
    for e0, e1 in sus_evs:
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    sus_map = dict(zip(sus_timed, sus_evs))
    t0 = time.perf_counter()
    for s_ in range(n_sus):
        for i, (_, _, a, w) in enumerate(ops):
            if i == dom and s_ in sus_map:
                _gemm.matmul_timed(a, w, *sus_map[s_])
            else:
                bi.matmul(a, w)
    torch.cuda.synchronize()
    sus_elapsed = time.perf_counter() - t0
    sus_us = [e0.elapsed_time(e1) * 1e3 for e0, e1 in sus_evs]
    q4 = sus_us[len(sus_us) * 3 // 4:]

    progress("per-shape")
    # Per-shape and stock comparison (HIP events, interleaved A/B, median of 9).
    def time_us(fn, reps=20):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    per_shape = []
    for (K, N), (_, _, a, w) in zip(SHAPES, ops):
        bi_t, st_t = [], []
        for _ in range(9):
            bi_t.append(time_us(lambda: bi.matmul(a, w)))
            st_t.append(time_us(lambda: torch.matmul(a, w)))
        tb, ts = statistics.median(bi_t), statistics.median(st_t)
        ratio = statistics.median(s_ / b_ for b_, s_ in zip(bi_t, st_t))
        per_shape.append({"M": M, "K": K, "N": N, "bi_us": round(tb, 2),
                          "speedup_vs_stock": round(ratio, 3),
                          "bi_tflops": round(gemm_flops(M, K, N) / tb / 1e6, 1),
                          "stock_us": round(ts, 2),
                          "stock_tflops": round(gemm_flops(M, K, N) / ts / 1e6, 1),
                          "roofline": gemm_roof(M, K, N, tb),
                          "geometry": _gemm.geometries()[
                              _gemm._lib.lib().bi_gemm_pick_geometry(M, N, K, 2, 0)]})

    progress("f16/fp32 sweep")
    # The same sweep in f16 and fp32 (fp32 against its own MFMA peak): HIP
    # events around whole steps, after a warmup.
    other_dtypes = {}
    for dname, dt in (("f16", torch.float16), ("f32", torch.float32)):
        ops_d = make_inputs(torch, dev, dt)
        for _ in range(3):
            for _, _, a, w in ops_d:
                bi.matmul(a, w)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        nrep = 10
        e0.record()
        for _ in range(nrep):
            for _, _, a, w in ops_d:
                bi.matmul(a, w)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / nrep
        tf = step_flops / ms / 1e9
        other_dtypes[dname] = {"ms_per_step": round(ms, 4), "tflops": round(tf, 1),
                               "mfma_frac": round(tf / PEAK_TFLOPS[dname], 4),
                               "peak_tflops": PEAK_TFLOPS[dname]}
        del ops_d
    torch.cuda.empty_cache()

    # Roofline of the dominant kernel: AI below the bf16 ridge, so HBM binds.
    Kd, Nd = DOMINANT
    fl, by = gemm_flops(M, Kd, Nd), gemm_bytes(M, Kd, Nd)
    hbm_achieved = by / dom_us / 1e3  # GB/s
    roof = {"bound": "hbm", "achieved": round(hbm_achieved, 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(hbm_achieved / PEAK_HBM_GBS, 4),
            "traffic": load_traffic(),
            "kernel": "bi_gemm bf16 %dx%dx%d (K,N) layout" % (M, Kd, Nd),
            "avg_launch_us": round(dom_us, 2),
            "launches_timed": len(evs),
            "mfma_achieved_tflops": round(fl / dom_us / 1e6, 1),
            "mfma_frac": round(fl / dom_us / 1e6 / PEAK_BF16_TFLOPS, 4),
            "frac_of_min_roof": round((fl / dom_us / 1e6) /
                                      min(PEAK_BF16_TFLOPS, fl / by * PEAK_HBM_GBS / 1e3), 4),
            "sustained": {"seconds": round(sus_elapsed, 2), "steps": n_sus,
                          "value_tflops": round(step_flops * n_sus / sus_elapsed / 1e12, 2),
                          "avg_launch_us": round(statistics.mean(sus_us), 2),
                          "frac": round(by / statistics.mean(sus_us) / 1e3 / PEAK_HBM_GBS, 4),
                          "last_quarter_avg_launch_us": round(statistics.mean(q4), 2),
                          "last_quarter_frac": round(by / statistics.mean(q4) / 1e3 /
                                                     PEAK_HBM_GBS, 4),
                          "launches_timed": len(sus_us)}}

    progress("decode attention")
    # Decode SDPA.
    g = torch.Generator().manual_seed(0)
    B, H, Hkv, N, D = SDPA["B"], SDPA["H"], SDPA["Hkv"], SDPA["N"], SDPA["D"]
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16).to(dev)
    sc = 1.0 / math.sqrt(D)
    sd_bi = statistics.median(time_us(lambda: bi.scaled_dot_product_attention(q, k, v, scale=sc),
                                      reps=10) for _ in range(5))
    sd_st = statistics.median(time_us(lambda: torch.nn.functional.scaled_dot_product_attention(
        q, k, v, scale=sc, enable_gqa=True), reps=10) for _ in range(5))
    sbytes = sdpa_bytes(B, H, Hkv, N, D)
    sdpa = {"config": dict(SDPA, qL=1, dtype="bf16"), "bi_us": round(sd_bi, 1),
            "gbps": round(sbytes / sd_bi / 1e3, 1), "stock_us": round(sd_st, 1),
            "stock_gbps": round(sbytes / sd_st / 1e3, 1),
            "roofline": {"bound": "hbm", "achieved": round(sbytes / sd_bi / 1e3, 1),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(sbytes / sd_bi / 1e3 / PEAK_HBM_GBS, 4)}}
    del q, k, v
    # Decode sweep over configs[2]'s range: B in {1, 8, 64} x N in {2048, 8192}.
    sweep = []
    for Bd in (1, 8, 64):
        for Nd in (2048, 8192):
            qd = torch.randn(Bd, H, 1, D, generator=g).to(torch.bfloat16).to(dev)
            kd = torch.randn(Bd, Hkv, Nd, D, generator=g).to(torch.bfloat16).to(dev)
            vd = torch.randn(Bd, Hkv, Nd, D, generator=g).to(torch.bfloat16).to(dev)
            t_bi = statistics.median(time_us(lambda: bi.scaled_dot_product_attention(
                qd, kd, vd, scale=sc), reps=10) for _ in range(5))
            t_st = statistics.median(time_us(lambda: torch.nn.functional.scaled_dot_product_attention(
                qd, kd, vd, scale=sc, enable_gqa=True), reps=10) for _ in range(5))
            by_d = sdpa_bytes(Bd, H, Hkv, Nd, D)
            sweep.append({"B": Bd, "N": Nd, "bi_us": round(t_bi, 1),
                          "gbps": round(by_d / t_bi / 1e3, 1),
                          "hbm_frac": round(by_d / t_bi / 1e3 / PEAK_HBM_GBS, 4),
                          "stock_us": round(t_st, 1)})
            del qd, kd, vd
    sdpa["sweep"] = sweep
    progress("graph-timed decode")
    # Small batches, graph-timed: 20 calls captured in a HIP graph and
    # replayed, so the figure is device time (eager calls at these sizes are
    # bound by the host's per-call cost).
    graph_cells = []
    for Bd in (1, 2, 4, 8):
        for Nd in (2048, 8192):
            qd = torch.randn(Bd, H, 1, D, generator=g).to(torch.bfloat16).to(dev)
            kd = torch.randn(Bd, Hkv, Nd, D, generator=g).to(torch.bfloat16).to(dev)
            vd = torch.randn(Bd, Hkv, Nd, D, generator=g).to(torch.bfloat16).to(dev)
            t_g = graph_us(torch, lambda: bi.scaled_dot_product_attention(qd, kd, vd, scale=sc))
            by_d = sdpa_bytes(Bd, H, Hkv, Nd, D)
            graph_cells.append({"B": Bd, "N": Nd, "bi_us": round(t_g, 2),
                                "gbps": round(by_d / t_g / 1e3, 1),
                                "hbm_frac": round(by_d / t_g / 1e3 / PEAK_HBM_GBS, 4)})
            del qd, kd, vd
    sdpa["graph_timed"] = graph_cells

    progress("prefill attention")
    # Causal prefill attention (the query-row-blocked path of the same kernel):
    # B=1, 32/8 heads, D=128, 2048 query rows over 2048 keys.
    L = 2048
    qp = torch.randn(1, H, L, D, generator=g).to(torch.bfloat16).to(dev)
    kp = torch.randn(1, Hkv, L, D, generator=g).to(torch.bfloat16).to(dev)
    vp = torch.randn(1, Hkv, L, D, generator=g).to(torch.bfloat16).to(dev)
    pf_bi = statistics.median(time_us(lambda: bi.scaled_dot_product_attention(
        qp, kp, vp, scale=sc, mask="causal"), reps=5) for _ in range(5))
    pf_st = statistics.median(time_us(lambda: torch.nn.functional.scaled_dot_product_attention(
        qp, kp, vp, scale=sc, is_causal=True, enable_gqa=True), reps=5) for _ in range(5))
    pf_flops = 4 * H * L * L * D / 2  # QK^T and PV over the causal half
    pf_bytes = float(2 * H * L * D + 2 * 2 * Hkv * L * D) * 2  # q, out, k, v once each
    pf_roof = min(PEAK_BF16_TFLOPS, pf_flops / pf_bytes * PEAK_HBM_GBS / 1e3)
    prefill = {"config": dict(B=1, H=H, Hkv=Hkv, qL=L, N=L, D=D, mask="causal", dtype="bf16"),
               "bi_us": round(pf_bi, 1), "bi_tflops": round(pf_flops / pf_bi / 1e6, 1),
               "stock_us": round(pf_st, 1), "stock_tflops": round(pf_flops / pf_st / 1e6, 1),
               "roofline": {"bound": "mfma" if pf_roof >= PEAK_BF16_TFLOPS else "hbm",
                            "frac_of_min_roof": round(pf_flops / pf_bi / 1e6 / pf_roof, 4),
                            "mfma_frac": round(pf_flops / pf_bi / 1e6 / PEAK_BF16_TFLOPS, 4)}}

    progress("quantized linear")
    # Affine 4-bit quantized linear (group 64), 4096 x 4096 weight: decode and
    # M=256 rows; stock is dequantize + F.linear.
    wq = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16)
    qw, qs, qz = (t.to(dev) for t in bi.quantize(wq, 64, 4))
    quant = {"config": dict(N=4096, K=4096, bits=4, group_size=64, dtype="bf16")}
    for Mq in (1, 256):
        xq = torch.randn(Mq, 4096, generator=g).to(torch.bfloat16).to(dev)
        q_bi = statistics.median(time_us(lambda: bi.quantized_linear(xq, qw, qs, qz, 64, 4))
                                 for _ in range(5))
        q_st = statistics.median(time_us(lambda: torch.nn.functional.linear(
            xq, bi.dequantize(qw, qs, qz, 64, 4))) for _ in range(5))
        # Algorithmic bytes: activations, packed weight, scales and biases, output.
        q_bytes = float(Mq * 4096 * 2 + 4096 * 4096 // 2 + 2 * 4096 * (4096 // 64) * 2
                        + Mq * 4096 * 2)
        q_flops = 2.0 * Mq * 4096 * 4096
        q_roof = min(PEAK_BF16_TFLOPS, q_flops / q_bytes * PEAK_HBM_GBS / 1e3)
        # Device time as well: 20 calls captured in a HIP graph and replayed
        # (an eager call at M=1 is bound by the host's per-call cost).
        q_g = graph_us(torch, lambda: bi.quantized_linear(xq, qw, qs, qz, 64, 4))
        quant["M%d" % Mq] = {"bi_us": round(q_bi, 1), "stock_us": round(q_st, 1),
                             "gbps": round(q_bytes / q_bi / 1e3, 1),
                             "tflops": round(q_flops / q_bi / 1e6, 2),
                             "frac_of_min_roof": round(q_flops / q_bi / 1e6 / q_roof, 4),
                             "graph_us": round(q_g, 2),
                             "graph_frac_of_min_roof": round(q_flops / q_g / 1e6 / q_roof, 4)}

    progress("invariance check")
    # Invariance spot check: row 0 of every shape of the sweep across batch
    # sizes 1..256 (each batch size picks its own workgroup footprint).
    differing = 0
    for _, _, a, w in ops:
        ref = bits(bi.matmul(a[:1].contiguous(), w)[0])
        for b in (2, 3, 8, 16, 17, 33, 64, 65, 128, 255, 256):
            differing += int((bits(bi.matmul(a[:b].contiguous(), w)[0]) != ref).sum())

    progress("M=4096 GEMMs and feed probe")
    prefill_gemm = prefill_gemms(torch, bi, dev)
    prefill_gemm["feed_probe"] = feed_probe(torch, dev)
    if not args.no_model:
        progress("model determinism")
    model = None if args.no_model else model_determinism(torch, bi, dev)
    if not args.no_cpu:
        progress("CPU baseline")
    cpu = None if args.no_cpu else cpu_baseline(ops)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[1] GEMM sweep at M=256, bf16, bi.matmul (K,N) weights",
                   "M": M, "shapes_KN": SHAPES, "parallelism": "none (one GPU)"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "per_shape": per_shape,
        "sweep_other_dtypes": other_dtypes,
        "sdpa_decode": sdpa,
        "prefill_gemm_m4096": prefill_gemm,
        "sdpa_prefill": prefill,
        "quantized_linear": quant,
        "invariance_bits_differing_batch_1_to_256": differing,
        "model_determinism": model,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
