"""Benchmark of the catena MI355X hot path (one GPU).

Headline workload: bf16 GEMM M=N=K=4096, fp32
accumulate, bf16 output, NN row-major, fixed reduction order.  One "step" is
one launch of that GEMM on inputs already resident in HBM.  The same JSON line
carries, under "extra", the KV-cache decode attention (configs[3]: B=32,
H=32, D=128, L=4096) and the decode-shape GEMMs, each with its
own roofline, because BASELINE.json's metric names both GEMM TFLOP/s and
attention HBM GB/s, and the decoder block of configs[4] (prefill and greedy
decode timed separately).

Timing: W untimed warmup launches, then K launches bracketed by stream
synchronisation and HIP events recorded on the library's own stream (the
stream every kernel is launched on).  Inputs come from the library's seeded
device RNG.  The cpu_baseline leg times the CPU oracle (the reference's
sequential arithmetic restated in C, gcc -O2 -ffp-contract=off) on a bounded
sample of the same workload on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--only gemm|core|decoder|all] [--no-ceilings]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "catena-lang_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import catena_amd as ca  # noqa: E402

METRIC = "det. bf16 GEMM TFLOP/s (%MFMA peak); KV-cache decode attention HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# non-packed, non-fused f32 VALU issue: 256 CUs x 64 lane-ops per clock x 2.4 GHz
PEAK_VALU_F32_TFLOPS = 256 * 64 * 2.4e9 / 1e12
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` (or per call of a workload whose
    entry sums the kernels one call launches) from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-kernel calibrated), or None.  Read
    from the file, not measured in this run: counters need a profiler pass
    of their own."""
    try:
        with open(TRAFFIC_FILE) as f:
            d = json.load(f)
        k = d["kernels"][kernel]
        return int(k["fetch_kib_raw"] * 1024 * d["fetch_factor"] + k["write_kib_raw"] * 1024 * d["write_factor"])
    except (OSError, KeyError, ValueError):
        return None


class HipEvents:
    """hipEvent timing on a given stream through libamdhip64."""

    def __init__(self, stream: int):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.stream = ctypes.c_void_p(stream)
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(self.a)) == 0
        assert self.hip.hipEventCreate(ctypes.byref(self.b)) == 0

    def start(self):
        assert self.hip.hipEventRecord(self.a, self.stream) == 0

    def close(self):
        for e in (self.a, self.b):
            if e:
                self.hip.hipEventDestroy(e)
        self.a = self.b = ctypes.c_void_p()

    def stop_ms(self) -> float:
        assert self.hip.hipEventRecord(self.b, self.stream) == 0
        assert self.hip.hipEventSynchronize(self.b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), self.a, self.b) == 0
        return ms.value


def timed(fn, steps: int, warmup: int, ev: HipEvents) -> float:
    """Average ms per call of fn over `steps` calls after `warmup` calls."""
    for i in range(warmup):
        fn(i)
    ca.synchronize()
    ev.start()
    for i in range(steps):
        fn(i)
    ms = ev.stop_ms()
    ca.synchronize()
    return ms / steps


def per_launch_us(fn, launches: int, ev: HipEvents) -> dict:
    """Each launch bracketed by its own events (after the timed run):
    median / p10 / p90 in microseconds, the protocol's per-launch spread."""
    t = []
    for i in range(launches):
        ev.start()
        fn(i)
        t.append(ev.stop_ms() * 1e3)
    t = np.array(t)
    return {"median": round(float(np.median(t)), 2), "p10": round(float(np.percentile(t, 10)), 2),
            "p90": round(float(np.percentile(t, 90)), 2), "launches": launches}


def host_cpu() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "cpus_visible": len(os.sched_getaffinity(0))}


def output_hash(buf: ca.Buffer) -> str:
    import hashlib
    return hashlib.sha256(buf.read(np.uint8).tobytes()).hexdigest()[:16]


# ------------------------------------------------------------------ workloads
def bench_c1(steps: int, ev):
    """configs[0] (C1): the 256^3 f32 GEMM, U[-1,1] inputs from seeds 1 and 2,
    through the program ABI symbol program_matmul_2x2_via_mem called as the
    reference's libffi executor calls a generated program (Mem by value,
    output through a pointer; synchronous, the output allocated by the
    callee and freed by the caller).  Times whole calls on the host clock
    (allocation, launch, synchronisation) and, with HIP events, the kernel
    alone; checks bitwise run to run."""
    n = m = k = 256
    a, b = ca.Buffer(n * k * 4), ca.Buffer(k * m * 4)
    ca.fill_uniform_f32(a, n * k, 1, 0)
    ca.fill_uniform_f32(b, k * m, 2, 0)
    L = ca.lib()
    hashes, got = set(), None

    def call(i):
        nonlocal got
        out = ca.Mem()
        L.program_matmul_2x2_via_mem(a.mem, b.mem, n, m, k, n * k, k * m, n * m, ctypes.byref(out))
        if i < 10:
            got = ca.mem_to_array(out, np.uint32).reshape(n, m)
            hashes.add(output_hash_np(got))
        ca.mem_free(out)

    for i in range(10):
        call(i)
    t = []
    for i in range(steps):
        t0 = time.perf_counter()
        call(10 + i)
        t.append((time.perf_counter() - t0) * 1e6)
    c = ca.Buffer(n * m * 4)
    # the kernel alone: launches through the bare C entry point with its
    # arguments bound once, so that the host's per-call cost (~4-5 us through
    # the checked Python wrapper) stays below the kernel's own duration; the
    # status of the last call is checked after the timed run
    f = L.catena_mi355x_gemm_f32_exact
    fargs = (ctypes.c_void_p(a.ptr), ctypes.c_void_p(b.ptr), ctypes.c_void_p(c.ptr),
             ctypes.c_uint64(n), ctypes.c_uint64(m), ctypes.c_uint64(k))
    st = [0]

    def launch_exact(i):
        st[0] = f(*fargs)

    k_ms = timed(launch_exact, steps, 10, ev)
    ca.check(st[0])
    flop = 2.0 * n * m * k
    return {"workload": "C1: f32 GEMM 256^3 as the program matmul-2x2-via-mem (program ABI, "
                        "by-value Mem), U[-1,1] from seeds 1 / 2",
            "us_per_program_call": round(float(np.median(t)), 2),
            "kernel_us": round(k_ms * 1e3, 3),
            "kernel_GFLOP/s": round(flop / (k_ms * 1e-3) / 1e9, 1),
            "bitwise_run_to_run": len(hashes) == 1,
            "roofline": {"bound": "valu", "achieved": round(flop / (k_ms * 1e-3) / 1e12, 3),
                         "peak": PEAK_VALU_F32_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flop / (k_ms * 1e-3) / 1e12 / PEAK_VALU_F32_TFLOPS, 4),
                         "traffic": None,
                         "work": "2 flop per multiply-add, each one VALU lane-op (v_mul_f32 then "
                                 "v_add_f32: the reference's separately rounded chain, no packed or "
                                 "fused ops); peak = 256 CUs x 64 f32 lane-ops per clock x 2.4 GHz"},
            "bound": "VALU issue (33.5 Mflop, 786 KB: far below HBM time)",
            "inputs": (a.read(np.float32, (n, k)), b.read(np.float32, (k, m)), got)}


def output_hash_np(arr) -> str:
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest()[:16]


def bench_gemm(steps, warmup, ev):
    n = m = k = 4096
    a, b, c = ca.Buffer(n * k * 2), ca.Buffer(k * m * 2), ca.Buffer(n * m * 2)
    ca.fill_normal_bf16(a, n * k, 3, 0, 1.0)
    ca.fill_normal_bf16(b, k * m, 4, 0, 1.0)
    ca.gemm_bf16(a, b, c, n, m, k)
    h0 = output_hash(c)
    ms = timed(lambda i: ca.gemm_bf16(a, b, c, n, m, k), steps, warmup, ev)
    flop = 2.0 * n * m * k
    tflops = flop / (ms * 1e-3) / 1e12
    same = output_hash(c) == h0
    spread = per_launch_us(lambda i: ca.gemm_bf16(a, b, c, n, m, k), max(10, steps), ev)
    same = same and output_hash(c) == h0
    return {"ms": ms, "tflops": tflops, "flop": flop, "bitwise_run_to_run": same,
            "per_launch_us": spread, "inputs": (a, b)}


def bench_gemm_operand_bits(steps, warmup, ev, a, b):
    """The same 4096^3 launch (same instructions, same memory traffic) on
    operands of different bit patterns: N(0,1) (the headline inputs),
    N(0,1) keeping 3 mantissa bits, constant 1.0 and zeros.  MFMA power
    depends on the operand bits and the clock follows the power limit, so
    the spread of these times is the clock's share of the headline time
    (the cycles per launch are the same; a GRBM_GUI_ACTIVE counter pass over
    `--only gemm-bits` reads them).  The headline inputs are restored."""
    n = 4096
    c = ca.Buffer(n * n * 2)
    keep_a, keep_b = a.read(np.uint16), b.read(np.uint16)
    out = {}
    for mode in ("normal", "normal_3bit_mantissa", "ones", "zeros"):
        if mode == "normal":
            ca.mem_write(a.mem, keep_a)
            ca.mem_write(b.mem, keep_b)
        elif mode == "normal_3bit_mantissa":
            ca.mem_write(a.mem, keep_a & np.uint16(0xFFF0))
            ca.mem_write(b.mem, keep_b & np.uint16(0xFFF0))
        else:
            v = np.uint16(0x3F80 if mode == "ones" else 0)
            ca.mem_write(a.mem, np.full(n * n, v, np.uint16))
            ca.mem_write(b.mem, np.full(n * n, v, np.uint16))
        ms = timed(lambda i: ca.gemm_bf16(a, b, c, n, n, n), steps, warmup, ev)
        out[mode] = {"us_per_launch": round(ms * 1e3, 2), "TFLOP/s": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1)}
    ca.mem_write(a.mem, keep_a)
    ca.mem_write(b.mem, keep_b)
    return out


def bench_decode_gemm(steps, warmup, ev):
    """M=16 x (N=11008, K=4096) and (N=4096, K=11008).  Four
    weight copies per shape rotate so the 90 MB weights cannot sit in the
    256 MB Infinity Cache between launches."""
    res = {}
    M = 16
    copies = 4
    for (N, K) in [(11008, 4096), (4096, 11008)]:
        x = ca.Buffer(M * K * 2)
        ca.fill_normal_bf16(x, M * K, 7, 0, 1.0)
        ws = []
        for c in range(copies):
            w = ca.Buffer(K * N * 2)
            ca.fill_normal_bf16(w, K * N, 8, c, 0.02)
            ws.append(w)
        y = ca.Buffer(M * N * 2)
        call = lambda i: ca.gemm_bf16(x, ws[i % copies], y, M, N, K)  # noqa: E731
        call(0)
        h0 = output_hash(y)
        ms = timed(call, steps, warmup, ev)
        call(0)
        same = output_hash(y) == h0
        nbytes = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
        gbs = nbytes / (ms * 1e-3) / 1e9
        groups, _ = ca.gemm_bf16_decode_plan(M, N, K)
        res[f"N{N}_K{K}"] = {"us": ms * 1e3, "GB/s": gbs, "frac_hbm": gbs / PEAK_HBM_GBS,
                             "bytes_per_launch": nbytes, "k_groups": groups,
                             "bitwise_run_to_run": same,
                             "per_launch_us": per_launch_us(call, max(10, steps), ev),
                             "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                          "frac": round(gbs / PEAK_HBM_GBS, 4),
                                          "traffic": measured_traffic(f"decode_gemm_N{N}_K{K}")},
                             "inputs": (x.read(np.uint16, (M, K)), ws[0].read(np.uint16, (K, N)))}
        del ws
    return res


def bench_attention(steps, warmup, ev):
    B, H, L, D = 32, 32, 4096, 128
    q = ca.Buffer(B * H * D * 2)
    k = ca.Buffer(B * H * L * D * 2)
    v = ca.Buffer(B * H * L * D * 2)
    ca.fill_normal_bf16(q, B * H * D, 41, 0, 1.0)
    ca.fill_normal_bf16(k, B * H * L * D, 41, 1, 1.0)
    ca.fill_normal_bf16(v, B * H * L * D, 41, 2, 1.0)
    lens = ca.Buffer.from_array(np.full(B, L, np.uint32))
    o = ca.Buffer(B * H * D * 4)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    call = lambda i: ca.attn_decode_bf16(q, k, v, lens, o, B, H, L, D, scale)  # noqa: E731
    call(0)
    h0 = output_hash(o)
    ms = timed(call, steps, warmup, ev)
    nbytes = 2.0 * B * H * L * D * 2 + B * H * D * 2 + B * H * D * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    same = output_hash(o) == h0
    spread = per_launch_us(call, max(10, steps), ev)
    same = same and output_hash(o) == h0
    return {"us": ms * 1e3, "GB/s": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "bytes_per_launch": nbytes,
            "bitwise_run_to_run": same, "per_launch_us": spread, "inputs": (q, k, v)}


def bench_decoder(reps: int, ev):
    """configs[4] (C5): one Llama-style block, d=2048, 16 heads of 128, SwiGLU
    5632, RMSNorm, RoPE; vocab 32000 embedding and LM head (bf16, N(0, 0.02));
    batch 8: a 512-token prefill, then 128 greedy decode steps that feed each
    argmax back on the device.  Times the prefill and the 128-step loop
    separately (HIP events on the library stream), median over `reps`."""
    d, H, F, layers, V, B, T, steps = 2048, 16, 5632, 1, 32000, 8, 512, 128
    dec = ca.Decoder(d, H, F, layers, V, B, T + steps)
    dec.init_weights(seed=51, std=0.02)
    tokens = np.random.default_rng(51).integers(0, V, (B, T)).astype(np.uint32)
    tb = ca.Buffer.from_array(tokens)
    nxt = ca.Buffer(B * 4)
    out = ca.Buffer(steps * B * 4)
    pre, gen, hashes = [], [], set()
    for r in range(reps + 1):
        ca.synchronize()
        ev.start()
        dec.prefill(tb, B, T, nxt)
        p_ms = ev.stop_ms()
        ev.start()
        dec.generate(steps, out)
        g_ms = ev.stop_ms()
        if r > 0:  # the first repetition allocates the activations
            pre.append(p_ms)
            gen.append(g_ms)
        hashes.add(output_hash(out))
    p_ms, g_ms = float(np.median(pre)), float(np.median(gen))
    # state for the CPU baseline: host weights, and the caches of a prefill
    dec.prefill(tb, B, T, nxt)
    ca.synchronize()
    w = {"embed": dec.read(ca.DEC_EMBED, np.uint16).reshape(V, d),
         "w_lm": dec.read(ca.DEC_W_LM, np.uint16).reshape(d, V),
         "w_qkv": [dec.read(ca.DEC_W_QKV, np.uint16).reshape(d, 3 * d)],
         "w_o": [dec.read(ca.DEC_W_O, np.uint16).reshape(d, d)],
         "w_gu": [dec.read(ca.DEC_W_GU, np.uint16).reshape(d, 2 * F)],
         "w_down": [dec.read(ca.DEC_W_DOWN, np.uint16).reshape(F, d)]}
    state = {"weights": w, "B": B, "T": T, "H": H, "F": F, "L": T + steps,
             "kc": [dec.read(ca.DEC_K_CACHE, np.uint16).reshape(B, H, T + steps, 128)],
             "vc": [dec.read(ca.DEC_V_CACHE, np.uint16).reshape(B, H, T + steps, 128)],
             "next": nxt.read(np.uint32), "tokens": tokens}
    block_params = 4 * d * d + 3 * d * F
    head_params = 2 * V * d  # embedding + LM head
    prefill_flop = 2.0 * B * T * block_params + 2.0 * B * d * V
    kv_step = 2.0 * B * H * 128 * 2 * (T + steps / 2)  # K + V read per step, average length
    step_bytes = 2.0 * (block_params + d * V) + kv_step
    res = {
        "workload": "C5: d=2048, 16x128 heads, SwiGLU 5632, RMSNorm, RoPE, 1 block, vocab 32000 "
                    "(embedding + LM head), batch 8, 512-token prefill then 128 greedy steps",
        "prefill_ms": p_ms,
        "prefill_tokens_per_s": B * T / (p_ms * 1e-3),
        "prefill_gemm_tflops": prefill_flop / (p_ms * 1e-3) / 1e12,
        "decode_ms_per_step": g_ms / steps,
        "decode_tokens_per_s": B * steps / (g_ms * 1e-3),
        "decode_bytes_per_step": step_bytes,
        "decode_GB/s": step_bytes / (g_ms / steps * 1e-3) / 1e9,
        "decode_frac_hbm": step_bytes / (g_ms / steps * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "params": {"block": block_params, "embedding_and_head": head_params},
        "bitwise_run_to_run": len(hashes) == 1,
        "roofline_prefill": {"bound": "mfma", "achieved": round(prefill_flop / (p_ms * 1e-3) / 1e12, 1),
                             "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(prefill_flop / (p_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                             "traffic": None,
                             "work": "GEMM flop of the prefill (block projections at 4096 rows + "
                                     "LM head at 8 rows) over the whole prefill time"},
        "roofline_decode": {"bound": "hbm", "achieved": round(step_bytes / (g_ms / steps * 1e-3) / 1e9, 1),
                            "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(step_bytes / (g_ms / steps * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                            "traffic": None,
                            "work": "bf16 weights (block + LM head) + K/V read per step (average "
                                    "cache length) over the step time"},
        "state": state,
    }
    dec.close()
    return res


# ------------------------------------------------------------------ CPU baseline
# The reference's arithmetic restated in C (oracle/, gcc -O2 -ffp-contract=off,
# kind "port") timed on this host's cores on a bounded sample of each
# workload: one warm-up call, then the median of CPU_RUNS timed calls, on all
# visible cores (<= 16) and on one thread.
CPU_RUNS = 5


def cpu_median_s(fn, runs: int = CPU_RUNS) -> float:
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_entry(value_fn, unit: str, threads: int, sample: str, single_sample: str,
              all_fn, single_fn) -> dict:
    """Median-of-CPU_RUNS timings of all_fn (on `threads` cores) and
    single_fn (one thread); value_fn(seconds, single) converts a time to the
    metric's unit for that sample."""
    t_all = cpu_median_s(all_fn)
    t_one = cpu_median_s(single_fn)
    return {"value": value_fn(t_all, False), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{sample}; median of {CPU_RUNS} runs {t_all:.3f} s",
            "median_of": CPU_RUNS,
            "single_thread": {"value": value_fn(t_one, True), "unit": unit, "cores": 1,
                              "sample": f"{single_sample}; median of {CPU_RUNS} runs {t_one:.3f} s"}}


def cpu_baseline_c1(a_host, b_host, got_bits, threads: int) -> dict:
    import oracle
    n, k = a_host.shape
    m = b_host.shape[1]
    want = oracle.matmul_f32(a_host, b_host, threads=threads)
    flop = 2.0 * n * m * k
    e = cpu_entry(lambda t, one: flop / t / 1e9, "GFLOP/s", threads,
                  f"the whole {n}x{m}x{k} f32 GEMM (sequential k-ascending fold)",
                  f"the whole {n}x{m}x{k} f32 GEMM",
                  lambda: oracle.matmul_f32(a_host, b_host, threads=threads),
                  lambda: oracle.matmul_f32(a_host, b_host, threads=1))
    e["gpu_bitwise_equal"] = bool(np.array_equal(got_bits, want.view(np.uint32)))
    return e


def cpu_baseline_gemm(a_buf, b_buf, threads: int) -> dict:
    import oracle
    n = k = m = 4096
    a16 = a_buf.read(np.uint16, (n, k))
    b16 = b_buf.read(np.uint16, (k, m))
    rows_all, rows_one = 512, 16
    sel_all = np.arange(rows_all, dtype=np.uint64)
    sel_one = np.arange(rows_one, dtype=np.uint64)
    return cpu_entry(lambda t, one: 2.0 * (rows_one if one else rows_all) * m * k / t / 1e12,
                     "TFLOP/s", threads,
                     f"{rows_all} of 4096 output rows of the 4096^3 bf16 GEMM, sequential "
                     f"k-ascending f32 fold (oracle/catena_oracle.c)",
                     f"{rows_one} of 4096 output rows",
                     lambda: oracle.matmul_bf16(a16, b16, rows=sel_all, threads=threads),
                     lambda: oracle.matmul_bf16(a16, b16, rows=sel_one, threads=1))


def cpu_baseline_decode_gemm(x16, w16, threads: int) -> dict:
    import oracle
    M, K = x16.shape
    N = w16.shape[1]
    nbytes = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
    rows_one = 4
    sel = np.arange(rows_one, dtype=np.uint64)
    # one thread on 4 of the 16 rows (the fold's cost is per output cell),
    # scaled to the whole launch's bytes
    return cpu_entry(lambda t, one: nbytes / (t * (M / rows_one if one else 1.0)) / 1e9, "GB/s",
                     threads, f"the whole M={M} x N={N} x K={K} decode GEMM",
                     f"{rows_one} of {M} rows, time scaled x{M // rows_one}",
                     lambda: oracle.matmul_bf16(x16, w16, threads=threads),
                     lambda: oracle.matmul_bf16(x16, w16, rows=sel, threads=1))


def cpu_baseline_attention(q, k, v, threads: int) -> dict:
    import oracle
    B, H, L, D = 32, 32, 4096, 128
    q16 = q.read(np.uint16, (B, H, D))
    n_all, n_one = 1024, 32

    def slices(nbh):
        kk = k.read(np.uint16, (nbh * L * D,)).reshape(1, nbh, L, D)
        vv = v.read(np.uint16, (nbh * L * D,)).reshape(1, nbh, L, D)
        return q16.reshape(1, B * H, D)[:, :nbh], kk, vv

    qa, ka, va = slices(n_all)
    lens = np.array([L], np.uint32)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    per = 2.0 * L * D * 2 + D * 2 + D * 4
    return cpu_entry(lambda t, one: (n_one if one else n_all) * per / t / 1e9, "GB/s", threads,
                     f"{n_all} of 1024 (batch, head) slices (sequential folds)",
                     f"{n_one} of 1024 slices",
                     lambda: oracle.attn_decode(qa, ka, va, lens, scale, threads=threads),
                     lambda: oracle.attn_decode(qa[:, :n_one], ka[:, :n_one], va[:, :n_one], lens,
                                                scale, threads=1))


def cpu_baseline_decoder(st: dict, threads: int) -> dict:
    """C5 on the oracle's whole-model sequential forward with the GPU model's
    weights: one greedy decode step at batch 8 from the GPU prefill's caches
    (cache length 512 -> 513), and the prefill of 8 tokens of one sequence."""
    from oracle import decoder as od
    w, kc, vc, nxt, tokens = st["weights"], st["kc"], st["vc"], st["next"], st["tokens"]
    B, T = st["B"], st["T"]
    mk = lambda th: od.DecoderOracle(w, st["H"], 128, st["F"], st["L"], threads=th)  # noqa: E731

    def step_fn(th, batch):
        o = mk(th)
        o.load_cache([c[:batch] for c in kc], [c[:batch] for c in vc], T)
        # each call appends one position (513, 514, ...): the same work
        return lambda: o.step(nxt[:batch], batch)

    pre_t = 8

    def prefill_fn(th):
        o = mk(th)
        return lambda: o.prefill(tokens[:1, :pre_t], 1, pre_t)

    dec = cpu_entry(lambda t, one: (1 if one else B) / t, "tokens/s", threads,
                    f"one decode step, batch {B}, cache length {T} -> {T + 1}",
                    f"one decode step of one sequence (batch 1)", step_fn(threads, B),
                    step_fn(1, 1))
    pre = cpu_entry(lambda t, one: pre_t / t, "tokens/s", threads,
                    f"prefill of {pre_t} tokens of one sequence", f"prefill of {pre_t} tokens",
                    prefill_fn(threads), prefill_fn(1))
    return {"decode": dec, "prefill": pre}


def bench_ceilings(ev: HipEvents) -> dict:
    """Measured ceilings of the resources the hot kernels are bound by, from
    the measurement kernels in csrc/kernels/calibrate.hip (a code object the
    library itself never loads): bf16 MFMA throughput and clock on random
    operands (registers only, then fed from LDS at the bf16 GEMM's read
    ratio), HBM read rate with plain and with non-temporal loads, and the
    4096^2 bf16 C-store write rate."""
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p

    def ck(e, what):
        if e != 0:
            raise RuntimeError(f"{what}: hip error {e}")

    path = os.path.join(ca.LIB_DIR, "calibrate.co")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run `python catena-lang_amd/build.py` first")
    mod = vp()
    ck(hip.hipModuleLoad(ctypes.byref(mod), path.encode()), "hipModuleLoad calibrate.co")
    stream = vp(ca.stream())

    def kernel(name):
        f = vp()
        ck(hip.hipModuleGetFunction(ctypes.byref(f), mod, name.encode()), name)
        return f

    def launcher(f, grid, block, vals):
        argv = (vp * len(vals))(*[ctypes.cast(ctypes.pointer(v), vp) for v in vals])

        def go():
            ck(hip.hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, stream, argv, None), "launch")
        go.keep = (vals, argv)
        return go

    def time_us(go, warmup, launches):
        for _ in range(warmup):
            go()
        ca.synchronize()
        ev.start()
        for _ in range(launches):
            go()
        return ev.stop_ms() / launches * 1e3

    out = {}
    grid, block, iters = 256, 512, 400
    obuf, cyc = ca.Buffer(grid * block * 4), ca.Buffer(grid * (block // 64) * 16)
    flop = grid * (block // 64) * iters * 32 * 16 * 16 * 32 * 2
    for key, name in (("mfma_bf16_random_operands", "catena_calib_mfma_bf16"),
                      ("mfma_bf16_lds_fed", "catena_calib_mfma_lds_bf16")):
        go = launcher(kernel(name), grid, block,
                      [vp(obuf.ptr), vp(cyc.ptr), ctypes.c_int(iters), ctypes.c_uint32(0x9E3779B9)])
        us = time_us(go, 300, 100)
        c = cyc.read(np.uint64).astype(np.float64).reshape(-1, 2)
        clk = c[:, 0] / (c[:, 1] / 100e6) / 1e9
        out[key] = {"TFLOP/s": round(flop / us / 1e6, 1), "frac_of_peak": round(flop / us / 1e6 / PEAK_BF16_TFLOPS, 4),
                    "clock_GHz_median": round(float(np.median(clk)), 3), "us_per_launch": round(us, 2)}
    # the same LDS-fed loop with one wave per SIMD and 128 x 128 wave tiles
    # (64 MFMAs : 24 LDS reads per step, accumulators in AGPRs)
    grid4, block4, iters4 = 256, 256, 400
    obuf4, cyc4 = ca.Buffer(grid4 * block4 * 4), ca.Buffer(grid4 * (block4 // 64) * 16)
    flop4 = grid4 * (block4 // 64) * iters4 * 64 * 16 * 16 * 32 * 2
    go = launcher(kernel("catena_calib_mfma_lds_4w_bf16"), grid4, block4,
                  [vp(obuf4.ptr), vp(cyc4.ptr), ctypes.c_int(iters4), ctypes.c_uint32(0x9E3779B9)])
    us = time_us(go, 300, 100)
    c = cyc4.read(np.uint64).astype(np.float64).reshape(-1, 2)
    clk = c[:, 0] / (c[:, 1] / 100e6) / 1e9
    out["mfma_bf16_lds_fed_4w_128x128"] = {
        "TFLOP/s": round(flop4 / us / 1e6, 1), "frac_of_peak": round(flop4 / us / 1e6 / PEAK_BF16_TFLOPS, 4),
        "clock_GHz_median": round(float(np.median(clk)), 3),
        "cycles_per_mfma_per_wave": round(float(np.median(c[:, 0])) / (iters4 * 64), 2), "us_per_launch": round(us, 2)}
    del obuf4, cyc4
    nbytes = 2 << 30
    src, flag = ca.Buffer(nbytes), ca.Buffer(64)
    ca.fill_uniform_f32(src, nbytes // 4, 11, 0)
    rgrid = 4096
    go = launcher(kernel("catena_calib_read"), rgrid, 512,
                  [vp(src.ptr), ctypes.c_uint64(nbytes // 16 // rgrid), vp(flag.ptr), ctypes.c_uint32(0x12345678)])
    us = time_us(go, 5, 50)
    out["hbm_read"] = {"GB/s": round(nbytes / us / 1e3, 1), "bytes": nbytes, "us_per_launch": round(us, 2)}
    go = launcher(kernel("catena_calib_read_nt"), rgrid, 512,
                  [vp(src.ptr), ctypes.c_uint64(nbytes // 16 // rgrid), vp(flag.ptr), ctypes.c_uint32(0x12345678)])
    us = time_us(go, 5, 50)
    out["hbm_read_nt"] = {"GB/s": round(nbytes / us / 1e3, 1), "bytes": nbytes, "us_per_launch": round(us, 2)}
    del src
    cbytes = 4096 * 4096 * 2
    cbuf = ca.Buffer(cbytes)
    go = launcher(kernel("catena_calib_write_tile"), 256, 512, [vp(cbuf.ptr), ctypes.c_uint32(7)])
    us = time_us(go, 50, 200)
    out["c_store_4096sq_bf16"] = {"GB/s": round(cbytes / us / 1e3, 1), "bytes": cbytes, "us_per_launch": round(us, 2)}
    ck(hip.hipModuleUnload(mod), "hipModuleUnload")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # Back-to-back GEMMs cross a power-management transient: in kernel traces
    # the first ~15 launches take ~103-105 us, launches 20-50 122-133 us, and
    # the durations decay to 104-107 us over launches 100-130 and settle at
    # 101-103 us after ~150; 200 warmup launches (~23 ms) put the timed
    # region in the steady state.  Every launch is the full GEMM.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["gemm", "gemm-bits", "core", "decoder", "all"], default="all",
                    help="gemm: the headline GEMM only; gemm-bits: + the same GEMM on other "
                         "operand bit patterns; core: + decode attention and decode GEMMs; "
                         "decoder: + the C5 decoder only; all: everything")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the measured ceilings (MFMA on random operands, LDS-fed MFMA, "
                         "HBM read, C-store write), run after everything else")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also launch the plain copy kernel on 1 GiB (known traffic) three "
                         "times, for scaling FETCH_SIZE / WRITE_SIZE counter readings")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the GEMM would shard by output columns and attention by (batch, head)). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    ca.init(0)
    ev = HipEvents(ca.stream())
    print("[bench] bf16 GEMM 4096^3", file=sys.stderr, flush=True)
    g = bench_gemm(args.steps, args.warmup, ev)
    extra = {"roofline_traffic_source": "every roofline.traffic figure is read from "
                                        "profiles/hbm_traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE "
                                        "passes of their own, scaled by a copy kernel of known size), "
                                        "not measured in this run"}
    core = args.only in ("core", "all")
    dec = c1 = at = dg = None
    if args.only in ("gemm-bits", "all"):
        print("[bench] bf16 GEMM 4096^3 on other operand bit patterns", file=sys.stderr, flush=True)
        a0, b0 = g["inputs"]
        extra["gemm_operand_bits"] = bench_gemm_operand_bits(args.steps, args.warmup, ev, a0, b0)
    if args.only in ("decoder", "all"):
        print("[bench] decoder block C5 (prefill 8x512, 128 greedy steps)", file=sys.stderr,
              flush=True)
        dec = bench_decoder(3, ev)
        extra["decoder_c5"] = {k_: v for k_, v in dec.items() if k_ != "state"}
    if core:
        print("[bench] C1 f32 GEMM 256^3 through program_matmul_2x2_via_mem", file=sys.stderr,
              flush=True)
        c1 = bench_c1(max(20, args.steps // 5), ev)
        extra["c1_f32_gemm_program"] = {k_: v for k_, v in c1.items() if k_ != "inputs"}
        print("[bench] decode attention B32 H32 L4096 D128", file=sys.stderr, flush=True)
        at = bench_attention(max(5, args.steps // 5), max(2, args.warmup // 5), ev)
        print("[bench] decode GEMMs M=16", file=sys.stderr, flush=True)
        dg = bench_decode_gemm(max(20, args.steps), args.warmup, ev)
        extra.update({
            "decode_attention": {
                "workload": "B=32 H=32 D=128 L=4096 bf16 KV, f32 softmax/out, bitwise vs sequential oracle",
                "us_per_launch": at["us"], "GB/s": at["GB/s"], "bitwise_run_to_run": at["bitwise_run_to_run"],
                "per_launch_us": at["per_launch_us"],
                "roofline": {"bound": "hbm", "achieved": at["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": at["frac_hbm"],
                             "traffic": measured_traffic("catena_attn_decode_bf16_d128")},
                "bytes_per_launch": at["bytes_per_launch"]},
            "decode_gemm_m16": {k_: {kk: vv for kk, vv in v.items() if kk != "inputs"}
                                for k_, v in dg.items()},
        })
    if args.copy_calibration:
        nbytes = 1 << 30
        src, dst = ca.Buffer(nbytes), ca.Buffer(nbytes)
        ca.fill_uniform_f32(src, nbytes // 4, 5, 0)
        for _ in range(3):
            ca.copy_bytes(dst, src, nbytes)
        ca.synchronize()
        print(f"[bench] copy calibration: 3 x catena_copy_16b over {nbytes} B", file=sys.stderr,
              flush=True)
    if not args.no_ceilings:
        print("[bench] ceilings (calibrate.hip)", file=sys.stderr, flush=True)
        extra["ceilings"] = bench_ceilings(ev)
    ev.close()
    cpu = None
    if not args.no_cpu_baseline:
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        print(f"[bench] cpu baselines ({threads} threads and 1 thread, median of {CPU_RUNS})",
              file=sys.stderr, flush=True)
        a, b = g["inputs"]
        cpu = cpu_baseline_gemm(a, b, threads)
        extra["host_cpu"] = host_cpu()
        if core:
            a1, b1, got1 = c1["inputs"]
            extra["c1_f32_gemm_program"]["cpu_baseline"] = cpu_baseline_c1(a1, b1, got1, threads)
            q, k, v = at["inputs"]
            extra["decode_attention"]["cpu_baseline"] = cpu_baseline_attention(q, k, v, threads)
            for key, v_ in dg.items():
                x16, w16 = v_["inputs"]
                extra["decode_gemm_m16"][key]["cpu_baseline"] = cpu_baseline_decode_gemm(x16, w16, threads)
        if dec is not None:
            extra["decoder_c5"]["cpu_baseline"] = cpu_baseline_decoder(dec["state"], threads)

    tflops = g["tflops"]
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded device RNG, N(0,1) bf16)",
        "config": {"workload": "bf16 GEMM M=N=K=4096, fp32 accumulate, bf16 out, NN row-major, "
                               "fixed K order (BASELINE configs[1])",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "bitwise_run_to_run": g["bitwise_run_to_run"],
        "per_launch_us": g["per_launch_us"],
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("catena_gemm_bf16_k32_bf16out")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ca.shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
