#!/usr/bin/env python3
"""Benchmark of the quantized-native matmul on one MI355X: weight GB/s (% of HBM peak) for the
Q4_K GEMV 14336x4096 at M=1 (the `value`) and M=16, on seeded synthetic packed weights.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is one projection call through the public entry point `mxa_gemm`: Q8_K quantization of
the activations and the fused dequantize-and-multiply over the packed weight (for M <= 3 both in
one kernel; for M = 16 a quantization kernel, then the matmul kernel). The timed region replays a
HIP graph of exactly K captured steps (so Python launch overhead is not measured), bracketed by
synchronizations. Each step reads a different copy of the weight (the copies together exceed
1 GiB), so the 256 MB Infinity Cache cannot serve repeats: every weight byte comes from HBM.

Timing: `ms_per_step` is device time, HIP events recorded on the replay stream around the K-step
replay, divided by K. A GPU-side wait is queued before the first event, so the whole replay is
submitted before the timed interval starts and the host's submission cost stays out of it (it
would otherwise be spread over K steps and make the figure depend on K). The host wall time of a
separate replay of the same K steps, synchronization included, is `host_ms_per_step`.

roofline: the dominant kernel is the M=1 matmul kernel (it also quantizes x): every M=1 step is
exactly one launch of it, so its average launch duration is the event interval of the timed
replay divided by K (gaps between launches included); achieved = algorithmic bytes per launch /
that duration. For M=16 the matmul kernel alone (activations quantized beforehand) is timed the
same way in a graph of its own. `traffic` is the HBM bytes per launch from rocprofv3 counters,
read from profiles/*_traffic.json only when that file was measured on the current kernel sources
(its `sources_sha16` equals the hash of matricxon_amd/csrc/*), else null.

cpu_baseline: the reference's own C kernel `mx_gemm` (built from its sources into
oracle/_ref/libmx_ref.so) on the host cores, same weight: M=1 with all usable threads (the
reference's default, the `value`), M=1 on one thread, and M=16 with all threads; the median of
timed calls after two warm-up calls each (the pattern of tools/benchmark_kernels.py:44-57).
"""

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
N, K = 14336, 4096
Q4_K, Q6_K = 12, 14
SEED_W, SEED_X = 2, 1002


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(m: int) -> int:
    """Bytes one launch must move at minimum: the packed weight once, the fp32 activations and the
    fp32 outputs (weight + M*K*4 + M*N*4)."""
    return N * (K // 256) * 144 + m * K * 4 + m * N * 4


def weight_bytes() -> int:
    return N * (K // 256) * 144


def cpu_has_avx2() -> bool:
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f in flags for f in (" avx2", " fma", " f16c"))


def host_layout() -> str:
    """The host CPU's model, sockets, cores and NUMA nodes (lscpu), and the CPUs this process may
    use."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return (f"{info.get('Model name', '?')}; {info.get('Socket(s)', '?')} socket(s) x "
            f"{info.get('Core(s) per socket', '?')} cores x {info.get('Thread(s) per core', '?')} "
            f"threads, {info.get('NUMA node(s)', '?')} NUMA node(s); "
            f"{len(os.sched_getaffinity(0))} CPUs usable by this process")


def cpu_baseline(w_np, seconds: float):
    """The reference C kernel on the host, ~`seconds` of calls in all: M=1 on all usable threads
    (the reference's default thread count), M=1 on one thread, M=16 on all threads. Each leg: two
    warm-up calls, then the median of timed calls over its share of the time."""
    if not cpu_has_avx2():
        log("host CPU lacks AVX2/FMA/F16C: no CPU baseline")
        return None
    from matricxon_amd import synthetic as S
    from oracle.native import REF_LIB, OracleGemm, RefGemm, default_threads

    threads = default_threads()
    if REF_LIB.exists():
        impl, kind = RefGemm(), "reference"
    else:
        impl, kind = OracleGemm(), "port"
    # as on the GPU, rotate over copies larger than the host caches, so every call streams its
    # weight from DRAM
    copies = [w_np] + [w_np.copy() for _ in range(3)]

    def leg(m: int, n_threads: int, budget: float) -> tuple[float, int]:
        x = S.activations(m, K, seed=SEED_X + m)
        for i in range(2):
            impl.gemm(Q4_K, copies[i], x, N, K, n_threads)
        times = []
        start = time.perf_counter()
        while time.perf_counter() - start < budget and len(times) < 100000:
            c = copies[len(times) % len(copies)]
            t0 = time.perf_counter()
            impl.gemm(Q4_K, c, x, N, K, n_threads)
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    med1, n1 = leg(1, threads, 0.4 * seconds)
    med1_1t, n1_1t = leg(1, 1, 0.3 * seconds)
    med16, n16 = leg(16, threads, 0.3 * seconds)
    wb = weight_bytes()
    return {
        "value": round(wb / med1 / 1e9, 2),
        "unit": "weight GB/s",
        "cores": threads,
        "kind": kind,
        "rows_per_s": round(N / med1),
        "one_thread_value": round(wb / med1_1t / 1e9, 2),
        "m16_value": round(wb / med16 / 1e9, 2),
        "m16_rows_per_s": round(N / med16),
        "layout": host_layout(),
        "sample": f"Q4_K 14336x4096 through mx_gemm, 4 host copies rotated (132 MB): M=1 on "
                  f"{threads} threads {n1} calls, median {med1 * 1e3:.3f} ms; M=1 on 1 thread "
                  f"{n1_1t} calls, median {med1_1t * 1e3:.3f} ms; M=16 on {threads} threads "
                  f"{n16} calls, median {med16 * 1e3:.3f} ms",
    }


# GPU-side wait queued ahead of a timed replay (torch.cuda._sleep spins this many clock cycles,
# about a millisecond): the host submits the whole replay meanwhile, so the events around it time
# the device alone.
LEAD_CYCLES = 3_000_000


def replay_ms(graph) -> float:
    """HIP-event milliseconds of one replay of `graph` on the current stream, with the replay fully
    queued before the first event fires."""
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(LEAD_CYCLES)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def capture(fn, steps: int, warmup: int):
    """A HIP graph of fn(0) .. fn(steps - 1), after `warmup` eager calls and one untimed replay."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(steps):
                fn(i)
    torch.cuda.current_stream().wait_stream(s)
    graph.replay()
    torch.cuda.synchronize()
    return graph


def eager_us(fn, steps: int, warmup: int) -> float:
    """Device microseconds per call of `steps` eager calls of fn(i), queued behind a GPU-side wait
    long enough for the host to submit them all, so the events time the device alone. For library
    calls kept out of HIP graphs (a reduction may record memset nodes there)."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(LEAD_CYCLES * max(1, steps // 10))
    e0.record()
    for i in range(steps):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def vendor_ceilings(weights, copies: int, steps: int, warmup: int) -> dict:
    """Vendor (torch / ROCm) kernels over the same rotated weight bytes, timed like the GEMV: a
    device-to-device copy (graph replay; reads and writes the bytes), a sum of the bytes viewed as
    int32 (eager, behind a GPU-side wait) and an empty kernel (graph replay: the fixed cost of one
    launch). They bound from outside what one launch over these bytes achieves on this box."""
    import torch

    nbytes = weights[0].numel()
    dst = torch.empty_like(weights[0])
    copy_us = _graph_us(lambda i: dst.copy_(weights[i % copies]), steps, warmup)
    sums = [torch.zeros((), dtype=torch.int64, device=dst.device)]
    sum_us = eager_us(lambda i: sums.__setitem__(0, weights[i % copies].view(torch.int32).sum()),
                      steps, warmup)
    empty_us = _graph_us(lambda i: torch.cuda._sleep(0), steps, warmup)
    del dst
    return {
        "vendor_copy_us": round(copy_us, 3),
        "vendor_copy_read_gbs": round(nbytes / copy_us / 1e3, 1),
        "vendor_copy_read_write_gbs": round(2 * nbytes / copy_us / 1e3, 1),
        "vendor_sum_i32_us": round(sum_us, 3),
        "vendor_sum_i32_read_gbs": round(nbytes / sum_us / 1e3, 1),
        "empty_kernel_us": round(empty_us, 3),
    }


def eager_module_call(gemm, dev, weights, copies: int, steps: int, warmup: int) -> dict:
    """One eager call of a bfloat16 `DevicePackedLinear` (the reference's GPU layer dtype) on the
    headline weight at M=1, as the reference's decode makes it (batch_decode.py:70-87 ->
    llama.py:265-279): host microseconds per call (wall time of `steps` calls back to back, one
    synchronization at the end) and device microseconds per call (HIP events around `steps` calls
    queued behind a GPU-side wait). Beside it, the same call through the float32 kernel with the
    casts a float32-only library needs (x to float32, y to bfloat16: two more launches). Calls
    rotate over the weight copies, as the timed GEMV does."""
    import torch

    from matricxon_amd import synthetic as S
    from matricxon_amd.device_packed import DevicePackedLinear

    mods = [DevicePackedLinear(w, K, Q4_K, dtype=torch.bfloat16) for w in weights[:copies]]
    x = torch.from_numpy(S.activations(1, K, seed=2)).to(dev).to(torch.bfloat16).reshape(1, 1, K)

    def module(i):
        return mods[i % copies](x)

    def cast_path(i):
        y = gemm.matmul(Q4_K, weights[i % copies], x.reshape(1, K).to(torch.float32), N, K)
        return y.to(torch.bfloat16).reshape(1, 1, N)

    def host_us(fn) -> float:
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / steps

    same = torch.equal(module(0), cast_path(0))
    res = {
        "module_host_us": round(host_us(module), 2),
        "module_device_us": round(eager_us(module, steps, warmup), 2),
        "cast_path_host_us": round(host_us(cast_path), 2),
        "cast_path_device_us": round(eager_us(cast_path, steps, warmup), 2),
        "same_bits": bool(same),
        "call": "DevicePackedLinear(Q4_K 14336x4096, dtype=bfloat16)(x bf16 (1, 1, 4096))",
    }
    del mods
    return res


def _graph_us(fn, steps: int, warmup: int) -> float:
    """Device microseconds per step of a HIP-graph replay of `steps` calls of fn(i)."""
    graph = capture(fn, steps, warmup)
    us = replay_ms(graph) * 1e3 / steps
    del graph
    return us


def bench_configs(gemm, dev, steps: int, warmup: int) -> None:
    """The reference's benchmark configs 1-5 on seeded synthetic data; weights rotated over
    copies totalling > 1 GiB where one copy fits in the 256 MB MALL."""
    import torch

    from matricxon_amd import synthetic as S
    from matricxon_amd.quant_types import row_bytes

    def weights(t, n, k, seed):
        w = torch.from_numpy(S.packed_weight(t, n, k, seed=seed)).to(dev)
        c = max(1, math.ceil((1 << 30) / w.numel()) + 1) if w.numel() < (512 << 20) else 1
        return [w] + [w.clone() for _ in range(c - 1)]

    def report(name, us, wbytes, flops=None):
        d = {"config": name, "us": round(us, 2), "weight_gbs": round(wbytes / us / 1e3, 1),
             "pct_hbm": round(100 * wbytes / us / 1e3 / HBM_PEAK_GBS, 1)}
        if flops:
            d["tflops"] = round(flops / us / 1e6, 1)
        print(json.dumps(d), file=sys.stderr, flush=True)

    def gemv(name, t, n, k, ms, seed):
        ws = weights(t, n, k, seed)
        for m in ms:
            x = torch.from_numpy(S.activations(m, k, seed=seed + m)).to(dev)
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            us = _graph_us(lambda i: gemm.matmul(t, ws[i % len(ws)], x, n, k, out=y), steps, warmup)
            report(f"{name} M={m}", us, n * row_bytes(t, k), 2.0 * m * n * k)
        del ws

    def gemv_f32(name, t, n, k, ms, seed):
        ws = weights(t, n, k, seed)
        for m in ms:
            x = torch.from_numpy(S.activations(m, k, seed=seed + m)).to(dev)
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            us = _graph_us(lambda i: gemm.gemv_f32(t, ws[i % len(ws)], x, n, k, out=y), steps, warmup)
            report(f"{name} M={m} fp32 activations", us, n * row_bytes(t, k), 2.0 * m * n * k)
        del ws

    gemv("cfg1 Q8_0 4096x4096", 8, 4096, 4096, [1], 11)
    gemv("cfg2 Q4_K 14336x4096", 12, 14336, 4096, [1, 2, 3, 4, 8, 16], 12)
    gemv("cfg3 Q6_K 128256x4096", 14, 128256, 4096, [1, 16], 13)
    # the fp32-activation GEMV (x not quantized), decode sizes
    gemv_f32("cfg1 Q8_0 4096x4096", 8, 4096, 4096, [1], 11)
    gemv_f32("cfg2 Q4_K 14336x4096", 12, 14336, 4096, [1, 4], 12)
    gemv_f32("cfg3 Q6_K 128256x4096", 14, 128256, 4096, [1], 13)
    gemv_f32("IQ4_XS 4096x4096", 23, 4096, 4096, [1], 14)
    # q, k (Q4_K), v (Q6_K), o, gate, up (Q4_K), down (Q6_K)
    layer = [(12, 4096, 4096), (12, 1024, 4096), (14, 1024, 4096), (12, 4096, 4096),
             (12, 14336, 4096), (12, 14336, 4096), (14, 4096, 14336)]
    # four copies of the layer (556 MB > the 256 MB MALL), one per step in turn
    lw = [weights(t, n, k, 40 + i)[:4] for i, (t, n, k) in enumerate(layer)]
    for m in (1, 16):
        xs = {k: torch.from_numpy(S.activations(m, k, seed=50 + k)).to(dev) for k in (4096, 14336)}
        ys = [torch.empty((m, n), dtype=torch.float32, device=dev) for _, n, _ in layer]

        def layer_step(i):
            for j, (t, n, k) in enumerate(layer):
                gemm.matmul(t, lw[j][i % 4], xs[k], n, k, out=ys[j])
        wb = sum(n * row_bytes(t, k) for t, n, k in layer)
        report(f"cfg4 llama3-8b layer (7 projections) M={m}", _graph_us(layer_step, steps, warmup),
               wb, 2.0 * m * sum(n * k for _, n, k in layer))
        # the layer as the model issues it: q|k|v and gate|up share their input (one activation
        # quantization each; one launch per group for up to 4 tokens)
        qkv_out = torch.empty((m, 6144), dtype=torch.float32, device=dev)
        gu_out = torch.empty((m, 28672), dtype=torch.float32, device=dev)

        def layer_shared_step(i):
            gemm.matmul_multi([(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (0, 1, 2)],
                              xs[4096], out=qkv_out)
            gemm.matmul(layer[3][0], lw[3][i % 4], xs[4096], 4096, 4096, out=ys[3])
            gemm.matmul_multi([(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (4, 5)],
                              xs[4096], out=gu_out)
            gemm.matmul(layer[6][0], lw[6][i % 4], xs[14336], 4096, 14336, out=ys[6])
        report(f"cfg4 llama3-8b layer (q|k|v, o, gate|up, down) M={m}",
               _graph_us(layer_shared_step, steps, warmup), wb,
               2.0 * m * sum(n * k for _, n, k in layer))
        # with its producers: RMSNorm before q|k|v and before gate|up, silu(gate) * up before
        # down. Unfused: the torch ops, then the projections quantize their inputs; fused: the
        # producer kernels also write the Q8_K blocks the projections run on
        norm_w = torch.linspace(0.5, 1.5, 4096, device=dev)
        xr = xs[4096]

        def rms_torch(x):
            return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5) * norm_w

        def layer_torch_producers(i):
            h = rms_torch(xr)
            gemm.matmul_multi([(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (0, 1, 2)], h,
                              out=qkv_out)
            gemm.matmul(layer[3][0], lw[3][i % 4], xr, 4096, 4096, out=ys[3])
            h = rms_torch(xr)
            gate, up = gemm.matmul_multi([(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (4, 5)],
                                         h, out=gu_out)
            act = torch.nn.functional.silu(gate) * up
            gemm.matmul(layer[6][0], lw[6][i % 4], act, 4096, 14336, out=ys[6])

        def layer_fused_producers(i):
            _, ws = gemm.rms_norm_q8k(xr, norm_w, 1e-5)
            gemm.matmul_multi_q8k([(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (0, 1, 2)],
                                  ws, m, 4096, out=qkv_out)
            gemm.matmul(layer[3][0], lw[3][i % 4], xr, 4096, 4096, out=ys[3])
            _, ws = gemm.rms_norm_q8k(xr, norm_w, 1e-5)
            gate, up = gemm.matmul_multi_q8k(
                [(layer[j][0], lw[j][i % 4], layer[j][1]) for j in (4, 5)], ws, m, 4096, out=gu_out)
            _, ws = gemm.silu_mul_q8k(gate, up)
            gemm.matmul_q8k(layer[6][0], lw[6][i % 4], ws, None, ys[6], m, 4096, 14336)
        for label, fn in (("torch RMSNorm/SwiGLU", layer_torch_producers),
                          ("fused producers", layer_fused_producers)):
            report(f"cfg4 llama3-8b layer + {label} M={m}", _graph_us(fn, steps, warmup), wb,
                   2.0 * m * sum(n * k for _, n, k in layer))
        names = ["q", "k", "v", "o", "gate", "up", "down"]
        for j, (t, n, k) in enumerate(layer):
            if names[j] in ("k", "up"):  # same shapes as v (size) / gate
                continue
            us = _graph_us(lambda i: gemm.matmul(t, lw[j][i % 4], xs[k], n, k, out=ys[j]), steps, warmup)
            report(f"cfg4   {names[j]} {'Q4_K' if t == 12 else 'Q6_K'} {n}x{k} M={m}", us,
                   n * row_bytes(t, k), 2.0 * m * n * k)
    del lw
    for t, name, n in ((12, "cfg5 Q4_K 14336x4096", 14336), (23, "cfg5 IQ4_XS 4096x4096", 4096)):
        w = torch.from_numpy(S.packed_weight(t, n, 4096, seed=60 + t)).to(dev)
        for m in (512, 2048):
            x = torch.from_numpy(S.activations(m, 4096, seed=70 + m)).to(dev)
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            us = _graph_us(lambda i: gemm.matmul(t, w, x, n, 4096, out=y), max(3, steps // 10), 2)
            report(f"{name} prefill M={m}", us, n * row_bytes(t, 4096), 2.0 * m * n * 4096)


def prefill_eager(gemm, dev, steps: int) -> None:
    """Eager launches of the config 5 prefill calls (the same weights and activations as
    `--configs`), each call's mean time printed on stderr: the workload of the MFMA counter runs."""
    import torch

    from matricxon_amd import synthetic as S

    for t, name, n in ((12, "Q4_K 14336x4096", 14336), (23, "IQ4_XS 4096x4096", 4096)):
        w = torch.from_numpy(S.packed_weight(t, n, 4096, seed=60 + t)).to(dev)
        for m in (512, 2048):
            x = torch.from_numpy(S.activations(m, 4096, seed=70 + m)).to(dev)
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            gemm.matmul(t, w, x, n, 4096, out=y)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                gemm.matmul(t, w, x, n, 4096, out=y)
            torch.cuda.synchronize()
            us = (time.perf_counter() - t0) / steps * 1e6
            log(f"prefill {name} M={m}: {us:.1f} us per call (eager, {steps} calls), "
                f"{2.0 * m * n * 4096 / us / 1e6:.1f} TFLOP/s-equivalent")


def long_rows_eager(gemm, dev, steps: int) -> None:
    """Eager launches of the long-row batched decode against the 16-block one, on Q8_K blocks
    quantized once: the config 4 down projection (4096x14336, 56 blocks per row) in Q6_K and
    Q4_K at M=16 (`bstream_kernel`), its one-row decode, and Q4_K 14336x4096 at M=16
    (`bwave_kernel`); each call's mean time printed on stderr. The workload of the counter runs
    that compare the two batched kernels' memory behaviour."""
    import torch

    from matricxon_amd import synthetic as S
    from matricxon_amd.gemm import q8k_bytes

    cases = ((14, "Q6_K 4096x14336", 4096, 14336, 16), (12, "Q4_K 4096x14336", 4096, 14336, 16),
             (14, "Q6_K 4096x14336", 4096, 14336, 1), (12, "Q4_K 14336x4096", 14336, 4096, 16))
    for t, name, n, k, m in cases:
        ws = [torch.from_numpy(S.packed_weight(t, n, k, seed=80 + t + c)).to(dev) for c in range(8)]
        x = torch.from_numpy(S.activations(m, k, seed=90 + m)).to(dev)
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        wsq = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device=dev)
        gemm.quantize_into(x, wsq)
        gemm.matmul_q8k(t, ws[0], wsq, None, y, m, n, k)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            gemm.matmul_q8k(t, ws[i % len(ws)], wsq, None, y, m, n, k)
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / steps * 1e6
        log(f"long rows {name} M={m}: {us:.1f} us per call (eager, {steps} calls, 8 weight copies)")
        del ws


def bench_load(dev) -> None:
    """Host -> HBM upload of the config 3 packed weight (128256 x 4096 Q6_K, 431 MB) from
    pageable host memory already in the page cache: the reference's `upload_packed`
    (frombuffer + `.to(device, copy=True)`) against `PackedUploader` (pinned, overlapped)."""
    import numpy as np
    import torch

    from matricxon_amd.loading import PackedUploader

    n, row = 128256, 3360
    raw = np.random.default_rng(7).integers(0, 256, n * row, dtype=np.uint8)
    mv = memoryview(raw)

    def timed(fn, reps=3):
        best = float("inf")
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
            del out
        return best

    t_ref = timed(lambda: torch.frombuffer(mv, dtype=torch.uint8).reshape(n, row)
                  .to(dev, copy=True))
    with PackedUploader(dev) as up:
        up.upload(mv, n)  # first use: pinned pages touched
        t_up = timed(lambda: up.upload(mv, n))
        got = up.upload(mv, n)
        ok = bool(torch.equal(got[::997].cpu(), torch.from_numpy(raw.reshape(n, row)[::997])))
    print(json.dumps({"config": "load Q6_K 128256x4096 host->HBM", "bytes": n * row,
                      "pageable_gbs": round(n * row / t_ref / 1e9, 1),
                      "staged_gbs": round(n * row / t_up / 1e9, 1), "rows_checked": ok}),
          file=sys.stderr, flush=True)


MOE_CASES = [
    # (name, n_experts, top_k, n_embd, ffn_len, types gate/up/down)
    ("mixtral-8x7b-like", 8, 2, 4096, 14336, (Q4_K, Q4_K, Q6_K)),
    ("granite-moe-3b-like", 40, 8, 1536, 512, (Q4_K, Q4_K, Q6_K)),
    ("olmoe-1b-7b-like", 64, 8, 2048, 1024, (Q4_K, Q4_K, Q6_K)),
]


def bench_moe(dev, steps: int) -> None:
    """One MoE expert FFN (moe_experts.py:81-88) on random-init packed experts, per token count:
    the grouped module (three launches for all experts, routing sorted on the device) against the
    reference's loop over per-expert DevicePackedLinear calls (one host sync on the routed ids,
    three calls per active expert). Both give the same bits (tests/test_gpu_moe.py). Eager wall
    time per forward; one JSON line per case on stderr."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from matricxon_amd import synthetic as S
    from matricxon_amd.device_packed import DevicePackedLinear
    from matricxon_amd.moe import HipPackedMoEExperts

    for name, n_exp, top_k, n_embd, ffn, types in MOE_CASES:
        raws = [np.concatenate([S.packed_weight(t, n_out, k_in, seed=100 * j + e)
                                for e in range(n_exp)])
                for j, (t, n_out, k_in) in enumerate(((types[0], ffn, n_embd),
                                                      (types[1], ffn, n_embd),
                                                      (types[2], n_embd, ffn)))]
        mod = HipPackedMoEExperts.from_packed_bytes(*(r.tobytes() for r in raws), types, n_exp,
                                                    n_embd, ffn, F.silu, torch.bfloat16, dev)
        per = [tuple(DevicePackedLinear(w[e], k_in, t, None, torch.bfloat16)
                     for w, k_in, t in ((mod.gate_packed, n_embd, types[0]),
                                        (mod.up_packed, n_embd, types[1]),
                                        (mod.down_packed, ffn, types[2])))
               for e in range(n_exp)]

        def loop(x, tw, tidx):
            out = torch.zeros(x.shape[0], n_embd, dtype=torch.float32, device=dev)
            for e in tidx.unique().tolist():
                g_m, u_m, d_m = per[e]
                tok, kk = (tidx == e).nonzero(as_tuple=True)
                x_e = x.index_select(0, tok).unsqueeze(0)
                h = F.silu(g_m(x_e)) * u_m(x_e)
                out.index_add_(0, tok, (d_m(h).squeeze(0) * tw[tok, kk].unsqueeze(-1)).float())
            return out.to(x.dtype)

        expert_bytes = sum(r.nbytes for r in raws) // n_exp
        for n_tok in (1, 16, 128):
            g = torch.Generator().manual_seed(n_tok)
            w, idx = torch.topk(torch.softmax(torch.randn(n_tok, n_exp, generator=g), -1), top_k)
            tw, tidx = (w / w.sum(-1, keepdim=True)).to(dev), idx.to(dev)
            x = torch.from_numpy(S.activations(n_tok, n_embd, seed=n_tok)).to(dev, torch.bfloat16)
            same = bool(torch.equal(mod(x, tw, tidx), loop(x, tw, tidx)))
            times = {}
            for label, fn in (("grouped", mod), ("per_expert_loop", loop)):
                for _ in range(3):
                    fn(x, tw, tidx)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(steps):
                    fn(x, tw, tidx)
                torch.cuda.synchronize()
                times[label] = (time.perf_counter() - t0) / steps * 1e6
            active = int(tidx.unique().numel())
            print(json.dumps({"config": f"moe {name} tokens={n_tok}", "experts": n_exp,
                              "top_k": top_k, "active_experts": active,
                              "grouped_us": round(times["grouped"], 1),
                              "per_expert_loop_us": round(times["per_expert_loop"], 1),
                              "speedup": round(times["per_expert_loop"] / times["grouped"], 2),
                              "grouped_weight_gbs": round(active * expert_bytes
                                                          / times["grouped"] / 1e3, 1),
                              "bit_identical": same}), file=sys.stderr, flush=True)
        del mod, per, raws
        torch.cuda.empty_cache()


def sources_sha16(files: tuple[str, ...]) -> str:
    """Hash of the kernel sources a measurement depends on: the named files of
    matricxon_amd/csrc and every shared header there (*.hpp). The stamp ties a counter measurement
    to the kernels it was taken on."""
    import hashlib

    csrc = REPO / "matricxon_amd" / "csrc"
    h = hashlib.sha256()
    for f in sorted(csrc.iterdir()):
        if f.suffix == ".hpp" or f.name in files:
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def traffic_of(name: str) -> int | None:
    """HBM bytes per launch from profiles/<name>_traffic.json when it was measured on the current
    sources of its kernel; None (and a note on stderr) when it is missing or stale."""
    f = REPO / "profiles" / f"{name}_traffic.json"
    if not f.exists():
        log(f"traffic: {f.name} missing")
        return None
    d = json.loads(f.read_text())
    files = next(files for prof, _, _, _, files in TRAFFIC_KERNELS if prof == name)
    if d.get("sources_sha16") != sources_sha16(files):
        log(f"traffic: {f.name} was measured on other kernel sources: reported as null")
        return None
    return int(d["hbm_bytes_per_launch"])


def q8k_act_bytes(m: int, k: int) -> int:
    """Bytes of m rows of Q8_K activations as the matrix-core kernels read them: int8 values, one
    float scale and sixteen int16 sums per 256 values."""
    return m * (k + (k // 256) * (4 + 32))


HEAD_N = 128256
# Workloads of `--kernel-only [--head]` whose HBM traffic `--traffic-summary` reports:
# (profile name, kernel-name pattern, algorithmic bytes per launch, workload, kernel source files)
TRAFFIC_KERNELS = [
    ("gemv_wave_q4k_14336x4096_m1", r"gemv_wave_kernel<12, 16, true, ", algorithmic_bytes(1),
     "Q4_K 14336x4096, M=1, x quantized in the kernel (weight + fp32 x + fp32 y)",
     ("mxa_gemv_wave.hip",)),
    ("bwave_q4k_14336x4096_m16", r"bwave_kernel<12, ",
     weight_bytes() + q8k_act_bytes(16, K) + 16 * N * 4,
     "Q4_K 14336x4096, M=16, on Q8_K activations (weight + Q8_K x + fp32 y)",
     ("mxa_bwave.hip",)),
    ("q6k_head_128256x4096_m1", r"gemv_wave_kernel<14, 16, true, ", HEAD_N * 3360 + K * 4 + HEAD_N * 4,
     "Q6_K 128256x4096 (config 3 head), M=1 (weight + fp32 x + fp32 y)", ("mxa_gemv_wave.hip",)),
    ("q6k_head_128256x4096_m16", r"bwave_kernel<14, ",
     HEAD_N * 3360 + q8k_act_bytes(16, K) + 16 * HEAD_N * 4,
     "Q6_K 128256x4096 (config 3 head), M=16, on Q8_K activations",
     ("mxa_bwave.hip",)),
]


def kernel_only_head(gemm, dev, steps: int) -> None:
    """Eager launches of the config 3 head's matmul kernel at M=1 and M=16 (431 MB, larger than
    the MALL on its own), for counter runs."""
    import torch

    from matricxon_amd import synthetic as S
    from matricxon_amd.gemm import q8k_bytes

    w = torch.from_numpy(S.packed_weight(14, HEAD_N, K, seed=13)).to(dev)
    for m in (1, 16):
        x = torch.from_numpy(S.activations(m, K, seed=13 + m)).to(dev)
        y = torch.empty((m, HEAD_N), dtype=torch.float32, device=dev)
        ws = torch.empty(q8k_bytes(m, K), dtype=torch.uint8, device=dev)
        fused = gemm.workspace_bytes(14, m, K) == 0
        if not fused:
            gemm.quantize_into(x, ws)
        for _ in range(steps):
            if fused:
                gemm.matmul(14, w, x, HEAD_N, K, out=y)
            else:
                gemm.matmul_q8k(14, w, ws, None, y, m, HEAD_N, K)
        torch.cuda.synchronize()
        log(f"head M={m}: {steps} launches")


def _pmc_values(directory: str, counter: str) -> dict[str, list[float]]:
    """Values of `counter` per kernel name, one per dispatch, from a rocprofv3 --pmc CSV output
    directory."""
    import csv

    vals: dict[str, list[float]] = {}
    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {directory}")
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") == counter:
                    vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return vals


def traffic_summary(fetch_dir: str, write_dir: str, cal_mib: int) -> int:
    """Counter passes -> profiles/<name>_traffic.json plus a Markdown table on stdout. Each counter
    is scaled by true / counted bytes of the calibration copy (the copy kernel with the largest
    reading: cal_mib MiB read and written)."""
    import re

    if cal_mib <= 0:
        raise SystemExit("--traffic-summary needs --calibrate-copy MIB (the calibration size)")
    fetch, write = _pmc_values(fetch_dir, "FETCH_SIZE"), _pmc_values(write_dir, "WRITE_SIZE")
    true_kib = cal_mib * 1024.0

    def scale(vals: dict[str, list[float]]) -> tuple[float, str]:
        # the calibration copy: the largest copy dispatches (the same copy kernel also moves the
        # smaller weight uploads and clones, which are not calibrations)
        copies = [(v, k) for k, vs in vals.items() if "copy" in k.lower() for v in vs]
        if not copies:
            raise SystemExit("no calibration copy kernel in the counter output")
        top = max(v for v, _ in copies)
        cal = [v for v, _ in copies if v >= 0.95 * top]
        return true_kib / (sum(cal) / len(cal)), max(copies)[1]

    fscale, fname = scale(fetch)
    wscale, wname = scale(write)
    print("| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes per launch | "
          "algorithmic bytes | ratio |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    print(f"| calibration `{fname[:40]}` ({cal_mib} MiB copy) | | scale {fscale:.4f} | "
          f"scale {wscale:.4f} | | | |")
    for prof, pattern, alg, workload, files in TRAFFIC_KERNELS:
        fk = [v for k, vs in fetch.items() if re.search(pattern, k) for v in vs]
        wk = [v for k, vs in write.items() if re.search(pattern, k) for v in vs]
        if not fk or not wk:
            continue
        names = sorted(k for k in fetch if re.search(pattern, k))
        f_kib, w_kib = sum(fk) / len(fk), sum(wk) / len(wk)
        hbm = round((f_kib * fscale + w_kib * wscale) * 1024)
        m = re.search(r"(\w+<[^<>]*>)\(", names[0])
        d = {"kernel": m.group(1) if m else names[0], "workload": workload,
             "hbm_bytes_per_launch": hbm, "fetch_kib": round(f_kib, 1),
             "write_kib": round(w_kib, 1), "fetch_scale": round(fscale, 4),
             "write_scale": round(wscale, 4), "dispatches": len(fk),
             "algorithmic_bytes": alg, "ratio": round(hbm / alg, 4),
             "sources_sha16": sources_sha16(files), "sources": list(files)}
        (REPO / "profiles" / f"{prof}_traffic.json").write_text(json.dumps(d, indent=1) + "\n")
        print(f"| `{d['kernel']}` ({workload}) | {d['dispatches']} | "
              f"{f_kib:.1f} | {w_kib:.1f} | {hbm} | {alg} | {hbm / alg:.3f} |")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=0, help="weight copies rotated (0: > 1 GiB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the per-launch kernel timing loop (for rocprofv3 --pmc runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only eager launches of the config 5 prefill calls (Q4_K 14336x4096 and "
                         "IQ4_XS 4096x4096 at M=512 and 2048; for rocprofv3 --pmc runs)")
    ap.add_argument("--long-only", action="store_true",
                    help="only eager launches of the config 4 down projection (56-block rows) at "
                         "M=16 and M=1 beside Q4_K 14336x4096 at M=16, on Q8_K blocks (for "
                         "rocprofv3 --pmc runs)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (scale for HBM counters)")
    ap.add_argument("--load", action="store_true",
                    help="also time the load path: the config 3 weight (431 MB) from host memory "
                         "into HBM, the reference's pageable copy vs the staged uploader")
    ap.add_argument("--configs", action="store_true",
                    help="also time the benchmark configs 1-5 (one JSON line each on stderr)")
    ap.add_argument("--moe", action="store_true",
                    help="only the MoE expert FFN: grouped launches vs the per-expert loop "
                         "(one JSON line per case on stderr)")
    ap.add_argument("--head", action="store_true",
                    help="with --kernel-only: also the config 3 Q6_K 128256x4096 head at M=1 "
                         "and M=16 (for rocprofv3 --pmc runs)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU work: read the rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE CSVs of "
                         "a --kernel-only [--head] --calibrate-copy MIB run, write "
                         "profiles/<kernel>_traffic.json stamped with the kernel sources' hash, "
                         "and print the summary table")
    args = ap.parse_args()
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary, args.calibrate_copy)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the kernels shard by output rows)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from matricxon_amd import synthetic as S
    from matricxon_amd.gemm import HipGemm, q8k_bytes

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gemm = HipGemm.get()
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    if args.prefill_only:
        prefill_eager(gemm, dev, args.steps)
        return 0
    if args.long_only:
        long_rows_eager(gemm, dev, args.steps)
        return 0
    if args.moe:
        bench_moe(dev, min(args.steps, 50))
        return 0

    w_np = S.packed_weight(Q4_K, N, K, seed=SEED_W)
    w0 = torch.from_numpy(w_np).to(dev)
    copies = args.copies or math.ceil((1 << 30) / w0.numel()) + 1
    weights = [w0] + [w0.clone() for _ in range(copies - 1)]
    log(f"{copies} weight copies, {copies * w0.numel() / 2**20:.0f} MiB rotated")

    results = {}
    for m in (1, 16):
        x = torch.from_numpy(S.activations(m, K, seed=SEED_X + m)).to(dev)
        ws = torch.empty(q8k_bytes(m, K), dtype=torch.uint8, device=dev)
        y = torch.empty((m, N), dtype=torch.float32, device=dev)
        ref_y = gemm.matmul(Q4_K, w0, x, N, K).clone()

        fused = gemm.workspace_bytes(Q4_K, m, K) == 0  # the matmul kernel quantizes x itself

        def step(i: int) -> None:
            """One projection call through the public entry point (mxa_gemm)."""
            gemm.matmul(Q4_K, weights[i % copies], x, N, K, out=y)

        def kernel(i: int) -> None:
            """The matmul kernel alone (the same call as `step` when that kernel quantizes x)."""
            if fused:
                gemm.matmul(Q4_K, weights[i % copies], x, N, K, out=y)
            else:
                gemm.matmul_q8k(Q4_K, weights[i % copies], ws, None, y, m, N, K)

        if not fused:
            gemm.quantize_into(x, ws)
        if args.kernel_only:  # eager launches only, for counter-collection runs
            for i in range(args.steps):
                kernel(i)
            torch.cuda.synchronize()
            if not torch.equal(y, ref_y):
                raise SystemExit(f"M={m}: kernel-only result differs from the full call")
            results[m] = {"launches": args.steps}
            continue

        def check(what: str) -> None:
            if not torch.equal(y, ref_y):
                raise SystemExit(f"M={m}: {what} result differs from the eager call")

        # -- timed region: a graph of exactly K steps ------------------------------------
        graph = capture(step, args.steps, args.warmup)
        check("graph replay")
        torch.cuda.synchronize()  # host wall time of one replay, synchronization included
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        host_ms = (time.perf_counter() - t0) * 1e3
        ev_ms = replay_ms(graph)  # the timed replay: device time of exactly K steps
        check("timed replay")
        del graph
        ms_step = ev_ms / args.steps
        kern_us = ms_step * 1e3
        if not fused:  # the matmul kernel alone in a graph of its own
            graph = capture(kernel, args.steps, args.warmup)
            kern_us = replay_ms(graph) * 1e3 / args.steps
            check("kernel-only replay")
            del graph
        results[m] = {
            "ms_per_step": ms_step,
            "host_ms_per_step": host_ms / args.steps,
            "weight_gbs": weight_bytes() / (ms_step * 1e-3) / 1e9,
            "rows_per_s": N / (ms_step * 1e-3),
            "kernel_us": kern_us,
            "kernel_weight_gbs": weight_bytes() / (kern_us * 1e-6) / 1e9,
            "kernel_alg_gbs": algorithmic_bytes(m) / (kern_us * 1e-6) / 1e9,
        }
        log(f"M={m}: {ms_step * 1e3:.2f} us/step (device; host {host_ms * 1e3 / args.steps:.2f}), "
            f"{results[m]['weight_gbs']:.0f} weight GB/s; matmul kernel {kern_us:.2f} us/launch, "
            f"{results[m]['kernel_alg_gbs']:.0f} GB/s algorithmic")

    if args.kernel_only and args.head:
        kernel_only_head(gemm, dev, args.steps)

    # The read floor: one launch of this library that only reads the same 33 MB
    # (mxa_stream_read), over the same rotated copies, timed the same way; beside it, vendor
    # kernels over the same bytes (a copy, an int32 sum) and an empty launch.
    floor_us, vendor = None, {}
    if not args.kernel_only:
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        floor_us = _graph_us(lambda i: gemm.stream_read(weights[i % copies], sink), args.steps,
                             args.warmup)
        log(f"read floor: {floor_us:.2f} us/launch for the same bytes, "
            f"{weight_bytes() / floor_us / 1e3:.0f} GB/s")
        vendor = vendor_ceilings(weights, copies, args.steps, args.warmup)
        log(f"vendor kernels over the same bytes: copy {vendor['vendor_copy_us']:.2f} us "
            f"({vendor['vendor_copy_read_gbs']:.0f} GB/s read), int32 sum "
            f"{vendor['vendor_sum_i32_us']:.2f} us ({vendor['vendor_sum_i32_read_gbs']:.0f} GB/s), "
            f"empty launch {vendor['empty_kernel_us']:.2f} us")

    eager = None
    if not args.kernel_only:
        eager = eager_module_call(gemm, dev, weights, copies, args.steps, args.warmup)
        log(f"eager bf16 module call, M=1: host {eager['module_host_us']:.1f} us, device "
            f"{eager['module_device_us']:.2f} us per call (float32 kernel + casts: host "
            f"{eager['cast_path_host_us']:.1f}, device {eager['cast_path_device_us']:.2f}); "
            f"same bits: {eager['same_bits']}")

    if args.configs:
        bench_configs(gemm, dev, max(20, args.steps // 4), args.warmup)

    if args.load:
        bench_load(dev)

    if args.calibrate_copy:
        nbytes = args.calibrate_copy << 20
        a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copy calibration: {nbytes} bytes read and written per copy kernel")

    if args.kernel_only:
        print(json.dumps({"kernel_only": True, **{f"m{m}": r for m, r in results.items()}}))
        return 0

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w_np, args.cpu_seconds)

    traffic1 = traffic_of("gemv_wave_q4k_14336x4096_m1")
    traffic16 = traffic_of("bwave_q4k_14336x4096_m16")

    r1, r16 = results[1], results[16]
    line = {
        "metric": "weight GB/s (% of HBM peak) for Q4_K GEMV 14336x4096 at M=1 and M=16",
        "value": round(r1["weight_gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r1["ms_per_step"], 5),
        "host_ms_per_step": round(r1["host_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded packed Q4_K blocks, N(0,1) activations)",
        "config": {
            "workload": "Q4_K GEMV 14336x4096, M=1 (config 2); weights rotated over "
                        f"{copies} HBM copies",
            "type": "Q4_K", "N": N, "K": K, "M": 1,
            "pct_of_hbm_peak": round(100 * r1["weight_gbs"] / HBM_PEAK_GBS, 1),
            "rows_per_s": round(r1["rows_per_s"]),
            "m16_weight_gbs": round(r16["weight_gbs"], 1),
            "m16_pct_of_hbm_peak": round(100 * r16["weight_gbs"] / HBM_PEAK_GBS, 1),
            "m16_ms_per_step": round(r16["ms_per_step"], 5),
            "m16_host_ms_per_step": round(r16["host_ms_per_step"], 5),
            "m16_kernel_us": round(r16["kernel_us"], 3),
            "m16_kernel_alg_gbs": round(r16["kernel_alg_gbs"], 1),
            "m16_rows_per_s": round(r16["rows_per_s"]),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r1["kernel_alg_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r1["kernel_alg_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic1,
            "kernel": "gemv_wave_kernel<Q4_K, nb=16, fused Q8_K>",
            "kernel_us": round(r1["kernel_us"], 3),
            "bytes_per_launch": algorithmic_bytes(1),
            "m16_traffic": traffic16,
            "m16_kernel": "bwave_kernel<Q4_K> (after quantize_q8k_kernel)",
            # one launch that only reads the weight bytes (mxa_stream_read), timed the same way
            "read_floor_us": round(floor_us, 3),
            "read_floor_weight_gbs": round(weight_bytes() / floor_us / 1e3, 1),
            "read_floor_frac_of_peak": round(weight_bytes() / floor_us / 1e3 / HBM_PEAK_GBS, 4),
            "kernel_vs_floor": round(floor_us / r1["kernel_us"], 4),
            **vendor,
        },
        "cpu_baseline": cpu,
        "eager_bf16_call": eager,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
