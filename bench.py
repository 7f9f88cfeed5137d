#!/usr/bin/env python3
"""Throughput of the HIP tensor-ops kernels on one MI355X.

Step: one pass of the FP16 unary/fused elementwise
workload -- SiLU and tanh-GELU on [8192, 8192] f16 N(0,1) and SwiGLU
out = a * silu(b) on [4096, 16384] f16 N(0,1), seed 1 -- with every input
already resident in HBM. `value` is the step's algorithmic bytes (each input
read once, each output written once) over the wall time of K steps. The K
launches of each kernel run back to back between HIP events on the SDK
stream (the stream the kernels run on), which gives each kernel's average
launch duration; the dominant kernel's achieved GB/s against the 8 TB/s HBM
peak is `roofline`. Operands rotate over enough identical copies that no
launch is served from the 256 MB last-level cache.

The other BASELINE configs are timed per kernel the same way and reported
under "suite". The CPU baseline times the oracle (a single-threaded C
restatement of the reference's portable path) on a bounded slice of the same
workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-suite] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_GBPS = 8000.0  # MI355X HBM3E
# MI355X dense matrix peaks (TFLOP/s): f16 MFMA; f32 MFMA for the f32 path
MFMA_PEAK_TFLOPS = {"f16": 2500.0, "f32": 157.3}

# Algorithmic bytes and elements per call (each distinct input read once +
# each output written once).
CFG2 = {
    "silu_f16": (268_435_456, 67_108_864),
    "gelu_f16": (268_435_456, 67_108_864),
    "swiglu_f16": (402_653_184, 67_108_864),
}


class Hip:
    """HIP runtime calls used for timing (events on the SDK stream)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipMemsetAsync.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                                            ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e.value

    def record(self, event, stream):
        assert self.lib.hipEventRecord(event, stream) == 0

    def elapsed_ms(self, start, stop):
        ms = ctypes.c_float()
        assert self.lib.hipEventSynchronize(stop) == 0
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop) == 0
        return ms.value

    def memset(self, ptr, nbytes, stream):
        assert self.lib.hipMemsetAsync(ptr, 0, nbytes, stream) == 0


TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "tensor_ops_hbm_traffic.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (lines `traffic_bytes <kernel> <bytes>`: FETCH_SIZE and WRITE_SIZE of
    two rocprofv3 --pmc runs, each scaled by the same counter's reading for a
    copy of known size), or None when the summary has no line for it."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic_bytes" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


def cpu_baseline(rows_fraction=4):
    """Oracle (single thread) on the first 1/rows_fraction of each cfg2 tensor,
    median of 5 after 1 warmup; reported in the metric's unit (GB/s of the
    same algorithmic bytes)."""
    import numpy as np
    from oracle import Oracle
    orc = Oracle()
    x = orc.normal((8192 // rows_fraction, 8192), 1, 0, 0.0, 1.0)
    a = orc.normal((4096 // rows_fraction, 16384), 1, 1, 0.0, 1.0)
    b = orc.normal((4096 // rows_fraction, 16384), 1, 2, 0.0, 1.0)
    times = []
    for rep in range(6):
        t0 = time.perf_counter()
        orc.silu(x)
        orc.gelu(x)
        orc.silu_multiply(b, a)
        dt = time.perf_counter() - t0
        if rep:
            times.append(dt)
    med = statistics.median(times)
    step_bytes = sum(v[0] for v in CFG2.values()) / rows_fraction
    del np
    return {"value": round(step_bytes / med / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"oracle/liboracle.so (C restatement, -O3, 1 thread) on the first 1/"
                       f"{rows_fraction} of the rows of each cfg2 tensor: SiLU+GELU "
                       f"[{8192 // rows_fraction},8192], SwiGLU [{4096 // rows_fraction},16384]; "
                       f"median of 5 after 1 warmup = {med:.3f} s"),
            "cpu_model": _cpu_model(), "host_cores": os.cpu_count()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---- per-config kernel suite ------------------------------------------------

ROTATE_BYTES = 600 << 20  # traffic between two uses of the same buffers (> 256 MB MALL)


def suite(sdk, hip, stream, reps=20, rounds=3):
    """Each BASELINE config's kernels: `reps` back-to-back launches between
    two events on the SDK stream, average per launch; the best of `rounds`
    such batches is reported with all of them. Every launch rotates to the
    next of enough identical copies of its operands that >= 600 MB of other
    traffic separates two uses of the same bytes, so no operand is served
    from the 256 MB last-level cache. Beside each kernel, a plain contiguous
    copy moving the same number of bytes is timed the same way
    (`copy_same_bytes_us`, `pct_of_copy`): below ~256 MB a single launch's
    fixed cost (launch, first-load latency, drain) keeps even a copy well
    under the 8 TB/s peak, and this is the ceiling a kernel of that size can
    be held to."""
    import numpy as np
    from inference_c_amd import TensorView
    results = {}
    T = sdk.tensor

    def filled(dtype, shape, kind, seed, stream_id, a, b):
        t = T(dtype, shape)
        sdk.call("tensor_fill_" + kind, t, seed, stream_id, a, b)
        return t

    def timed(make_set, run, alg_bytes, warmup=3):
        copies = max(1, -(-ROTATE_BYTES // alg_bytes))
        sets = [make_set() for _ in range(copies)]
        for i in range(warmup):
            run(sets[i % copies])
        start, stop = hip.event(), hip.event()
        batches = []
        for _ in range(rounds):
            hip.record(start, stream)
            for i in range(reps):
                run(sets[i % copies])
            hip.record(stop, stream)
            batches.append(hip.elapsed_ms(start, stop) / reps)
        del sets
        sdk.synchronize()
        return batches, copies

    copy_floor = {}

    def copy_us(alg_bytes):
        """Best time of a plain contiguous f16 copy moving the same bytes
        (alg_bytes / 2 read, alg_bytes / 2 written): what one launch of this
        size reaches on this device, launch and drain included."""
        if alg_bytes not in copy_floor:
            n = alg_bytes // 4
            view = TensorView.make((n,), (1,), 0)
            batches, _ = timed(lambda: (filled("f16", (n,), "normal", 9, 0, 0.0, 1.0),
                                        T("f16", (n,))),
                               lambda c: sdk.call("tensor_view_add_mul_f16", c[0], view, None,
                                                  None, c[1]), alg_bytes)
            copy_floor[alg_bytes] = min(batches)
        return copy_floor[alg_bytes]

    def measure(name, make_set, run, alg_bytes, elements):
        batches, copies = timed(make_set, run, alg_bytes)
        best = min(batches)
        floor = copy_us(alg_bytes)
        results[name] = {"avg_us": round(best * 1e3, 2),
                         "batches_us": [round(t * 1e3, 2) for t in batches],
                         "gbps": round(alg_bytes / (best * 1e-3) / 1e9, 1),
                         "pct_peak": round(100 * alg_bytes / (best * 1e-3) / 1e9 / PEAK_GBPS, 1),
                         "elements_per_s": float(f"{elements / (best * 1e-3):.4g}"),
                         "bytes": alg_bytes, "buffer_sets": copies,
                         "copy_same_bytes_us": round(floor * 1e3, 2),
                         "pct_of_copy": round(100 * floor / best, 1)}

    # cfg1: f32 add / mul / row-bias add [1024, 4096], U[-1,1], seed 0
    def cfg1():
        return (filled("f32", (1024, 4096), "uniform", 0, 0, -1.0, 1.0),
                filled("f32", (1024, 4096), "uniform", 0, 1, -1.0, 1.0),
                filled("f32", (4096,), "uniform", 0, 2, -1.0, 1.0), T("f32", (1024, 4096)))
    measure("cfg1_add_f32", cfg1, lambda s: sdk.call("tensor_add_f32", s[0], s[1], s[3]),
            50_331_648, 4_194_304)
    measure("cfg1_mul_f32", cfg1, lambda s: sdk.call("tensor_mul_f32", s[0], s[1], s[3]),
            50_331_648, 4_194_304)
    measure("cfg1_bias_add_f32", cfg1, lambda s: sdk.call("tensor_bias_add_f32", s[0], s[2], s[3]),
            33_570_816, 4_194_304)
    # cfg2: SiLU / GELU [8192, 8192], SwiGLU [4096, 16384], f16 N(0,1), seed 1
    def cfg2_unary():
        return filled("f16", (8192, 8192), "normal", 1, 0, 0.0, 1.0), T("f16", (8192, 8192))
    measure("cfg2_silu_f16", cfg2_unary, lambda s: sdk.call("tensor_silu_f16", s[0], s[1]),
            *CFG2["silu_f16"])
    measure("cfg2_gelu_f16", cfg2_unary, lambda s: sdk.call("tensor_gelu_f16", s[0], s[1]),
            *CFG2["gelu_f16"])
    def cfg2_swiglu():
        return (filled("f16", (4096, 16384), "normal", 1, 1, 0.0, 1.0),
                filled("f16", (4096, 16384), "normal", 1, 2, 0.0, 1.0), T("f16", (4096, 16384)))
    measure("cfg2_swiglu_f16", cfg2_swiglu,
            lambda s: sdk.call("tensor_silu_multiply_f16", s[1], s[0], s[2]), *CFG2["swiglu_f16"])
    # cfg3: RMSNorm [16384, 2048]; causal softmax / row sum / row max on [32, 2048, 2048]
    def cfg3_rms():
        return (filled("f16", (16384, 2048), "normal", 3, 0, 0.0, 1.0),
                filled("f16", (2048,), "uniform", 3, 1, 0.5, 1.5), T("f16", (16384, 2048)))
    measure("cfg3_rms_norm_f16", cfg3_rms,
            lambda s: sdk.call("tensor_rms_norm_f16", s[0], s[1], 1e-6, s[2]), 134_221_824, 33_554_432)
    def cfg3_logits():
        return (filled("f16", (32, 2048, 2048), "normal", 3, 2, 0.0, 3.0), T("f16", (32, 2048, 2048)),
                T("f32", (32, 2048)))
    measure("cfg3_causal_softmax_f16", cfg3_logits,
            lambda s: sdk.call("tensor_softmax_f16", s[0], 1, s[1]), 536_870_912, 134_217_728)
    measure("cfg3_row_sum_f16", cfg3_logits, lambda s: sdk.call("tensor_row_sum_f16", s[0], s[2]),
            268_697_600, 134_217_728)
    measure("cfg3_row_max_f16", cfg3_logits, lambda s: sdk.call("tensor_row_max_f16", s[0], s[2]),
            268_697_600, 134_217_728)
    # cfg4: (x.permute(0,2,1,3) + A) * M, x [16,1024,32,64]
    B, S, H, D = 16, 1024, 32, 64
    view = TensorView.make((B, H, S, D), (S * H * D, D, H * D, 1), 0)
    def cfg4():
        return (filled("f16", (B, S, H, D), "normal", 4, 0, 0.0, 1.0),
                filled("f16", (1, H, 1, D), "uniform", 4, 1, -1.0, 1.0),
                filled("f16", (B, 1, S, 1), "uniform", 4, 2, -1.0, 1.0), T("f16", (B, H, S, D)))
    measure("cfg4_permuted_broadcast_f16", cfg4,
            lambda s: sdk.call("tensor_view_add_mul_f16", s[0], view, s[1], s[2], s[3]),
            134_254_592, 33_554_432)
    # cfg5: decoder chain (fused residual+RMSNorm, RoPE q+k, SwiGLU) timed as one chain
    tok, hid, inter = 4096, 2048, 8192
    def cfg5():
        return {"x": filled("f16", (tok, hid), "normal", 5, 0, 0.0, 1.0),
                "r": filled("f16", (tok, hid), "normal", 5, 1, 0.0, 1.0),
                "w": filled("f16", (hid,), "normal", 5, 9, 0.0, 1.0),
                "h": T("f16", (tok, hid)), "n": T("f16", (tok, hid)),
                "q": filled("f16", (tok, 32, 64), "normal", 5, 2, 0.0, 1.0),
                "k": filled("f16", (tok, 32, 64), "normal", 5, 3, 0.0, 1.0),
                "g": filled("f16", (tok, inter), "normal", 5, 4, 0.0, 1.0),
                "u": filled("f16", (tok, inter), "normal", 5, 5, 0.0, 1.0),
                "o": T("f16", (tok, inter))}
    def norm(s):
        sdk.call("tensor_residual_rms_norm_f16", s["x"], s["r"], s["w"], 1e-6, s["h"], s["n"])
    def rope(s):
        sdk.call("tensor_rope_f16", s["q"], s["k"], 32, 32, 64, 10000.0, 0)
    def swiglu(s):
        sdk.call("tensor_silu_multiply_f16", s["g"], s["u"], s["o"])
    def chain(s):
        norm(s)
        rope(s)
        swiglu(s)
    measure("cfg5_decoder_chain_f16", cfg5, chain, 335_548_416, 142_606_336)
    measure("cfg5_residual_rms_norm_f16", cfg5, norm, 67_112_960, 8_388_608)
    measure("cfg5_rope_f16", cfg5, rope, 67_108_864, 16_777_216)
    measure("cfg5_swiglu_f16", cfg5, swiglu, 201_326_592, 33_554_432)
    # embedding gather: a 32768-token prefill batch of int32 ids into
    # a [32000, 2048] f16 table; device storage, so each call also runs the
    # one-block index check and waits for its verdict before gathering
    vocab, width, tokens = 32000, 2048, 32768
    emb_table = filled("f16", (vocab, width), "normal", 6, 0, 0.0, 1.0)
    def gather_set():
        ids = T("i32", (tokens,))
        host_ids = ((np.arange(tokens, dtype=np.int64) * 2654435761) % vocab).astype(np.int32)
        ids.upload(host_ids)
        return ids, T("f16", (tokens, width))
    measure("embedding_lookup_f16", gather_set,
            lambda s: sdk.call("tensor_embedding_lookup_f16", emb_table, s[0], s[1]),
            2 * tokens * width * 2 + tokens * 4, tokens * width)
    del emb_table
    # quantized linear (HBM-bound on the packed weights): a [28672, 8192]
    # Q8_0 / Q4_0 matrix (a 70B-class MLP up+gate projection) times 1 or 4 f16
    # rows (the GEMV) or 16 rows (the MFMA kernel: small-batch decode);
    # synthetic packed bytes with an f16 scale of 2^-7
    rng = np.random.default_rng(7)
    def packed_weights(out, inw, block):
        raw = rng.integers(0, 256, size=(out, inw // 32, block), dtype=np.uint8)
        raw[:, :, 0:2] = np.frombuffer(np.float16(2.0 ** -7).tobytes(), np.uint8)
        return raw
    for fmt, block in (("q8_0", 34), ("q4_0", 18)):
        out_f, in_f = 28672, 8192
        host_w = packed_weights(out_f, in_f, block)
        for rows in ((1, 4, 16) if fmt == "q8_0" else (1,)):
            def quant_set(rows=rows, host_w=host_w):
                return (T("u8", host_w.shape).upload(host_w),
                        filled("f16", (rows, in_f), "normal", 7, 3, 0.0, 1.0),
                        T("f16", (rows, out_f)))
            measure(f"linear_{fmt}_f16_{rows}x{in_f}_to_{out_f}", quant_set,
                    lambda s, fmt=fmt: sdk.call(f"tensor_linear_{fmt}_f16", s[1], s[0], s[2]),
                    host_w.nbytes + rows * (in_f + out_f) * 2, rows * out_f)
        del host_w
    # f16 linear through hipBLASLt: a decode row (HBM-bound GEMV on the
    # weights) and a 4096-token prefill (MFMA-bound)
    def linear_set(rows, inw, out_f):
        return lambda: (filled("f16", (rows, inw), "normal", 8, 0, 0.0, 1.0),
                        filled("f16", (out_f, inw), "normal", 8, 1, 0.0, 0.02),
                        filled("f16", (out_f,), "normal", 8, 2, 0.0, 1.0), T("f16", (rows, out_f)))
    run_linear = lambda s: sdk.call("tensor_linear_f16", s[0], s[1], s[2], s[3])
    measure("linear_f16_decode_1x8192_to_8192", linear_set(1, 8192, 8192), run_linear,
            8192 * 8192 * 2 + 2 * 8192 * 2 + 8192 * 2, 8192)
    rows_p = in_p = out_p = 4096
    p_flops = 2.0 * rows_p * in_p * out_p
    p_bytes = (rows_p * in_p + out_p * in_p + rows_p * out_p + out_p) * 2
    batches, _ = timed(linear_set(rows_p, in_p, out_p), run_linear, p_bytes)
    best = min(batches)
    results["linear_f16_prefill_4096x4096_to_4096_bias"] = {
        "avg_us": round(best * 1e3, 2), "batches_us": [round(t * 1e3, 2) for t in batches],
        "tflops": round(p_flops / (best * 1e-3) / 1e12, 1),
        "pct_peak_mfma": round(100 * p_flops / (best * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["f16"], 1),
        "peak_tflops": MFMA_PEAK_TFLOPS["f16"], "flops": p_flops, "bytes": p_bytes,
        "library": "hipBLASLt (bias epilogue)"}
    # host-pointer compute-table slot (PCIe included, never `value`): SwiGLU
    # on cfg2's [4096, 16384] f16 operands in pageable host memory, staged
    # through the pinned chunk pool; wall clock of the synchronous call
    import ctypes as _ct
    table = sdk.compute_table()
    slot = _ct.CFUNCTYPE(_ct.c_int, _ct.c_void_p, _ct.c_void_p, _ct.c_void_p,
                         _ct.c_size_t)(table.silu_multiply_f16)
    n_host = 4096 * 16384
    ha = np.random.default_rng(1).standard_normal(n_host).astype(np.float16)
    hb = np.random.default_rng(2).standard_normal(n_host).astype(np.float16)
    hy = np.empty_like(ha)
    assert slot(ha.ctypes.data, hb.ctypes.data, hy.ctypes.data, n_host)
    walls = []
    for _ in range(5):
        t0 = time.perf_counter()
        assert slot(ha.ctypes.data, hb.ctypes.data, hy.ctypes.data, n_host)
        walls.append(time.perf_counter() - t0)
    wall = statistics.median(walls)
    results["host_slot_swiglu_f16_pcie"] = {
        "wall_us": round(wall * 1e6, 1), "bytes": 3 * 2 * n_host,
        "gbps_pcie_inclusive": round(3 * 2 * n_host / wall / 1e9, 2),
        "note": "inputs and output in pageable host memory; median of 5 synchronous calls"}
    del ha, hb, hy
    # attention (MFMA-bound, not HBM): scaled dot-product attention on device
    # buffers; flops = 4 * B * Hq * Lq * Lkv * D (half for causal), against
    # the 2.5 PFLOP/s dense f16 MFMA peak
    def measure_attention(name, b, hq, hkv, lq, lk, d, causal, dtype="f16"):
        def make():
            return (filled(dtype, (b, hq, lq, d), "normal", 7, 0, 0.0, 1.0),
                    filled(dtype, (b, hkv, lk, d), "normal", 7, 1, 0.0, 1.0),
                    filled(dtype, (b, hkv, lk, d), "normal", 7, 2, 0.0, 1.0),
                    T(dtype, (b, hq, lq, d)))
        flops = 4.0 * b * hq * lq * lk * d * (0.5 if causal else 1.0)
        size = 2 if dtype == "f16" else 4
        alg_bytes = (2 * b * hq * lq * d + 2 * b * hkv * lk * d) * size
        batches, copies = timed(make, lambda s: sdk.call(f"tensor_sdpa_device_{dtype}", s[0], s[1],
                                                         s[2], None, 1.0 / d ** 0.5, int(causal),
                                                         s[3]), alg_bytes)
        best = min(batches)
        peak = MFMA_PEAK_TFLOPS[dtype]
        results[name] = {"avg_us": round(best * 1e3, 2),
                         "batches_us": [round(t * 1e3, 2) for t in batches],
                         "tflops": round(flops / (best * 1e-3) / 1e12, 1),
                         "pct_peak_mfma": round(100 * flops / (best * 1e-3) / 1e12 / peak, 1),
                         "peak_tflops": peak, "flops": flops, "bytes": alg_bytes,
                         "shape": {"batch": b, "q_heads": hq, "kv_heads": hkv, "q_len": lq,
                                   "kv_len": lk, "head_dim": d, "causal": causal}}
    measure_attention("sdpa_f16_prefill_32q8kv_2048_d128_causal", 1, 32, 8, 2048, 2048, 128, True)
    measure_attention("sdpa_f16_vision_12h_1024_d64", 1, 12, 12, 1024, 1024, 64, False)
    measure_attention("sdpa_f32_12h_1024_d64", 1, 12, 12, 1024, 1024, 64, False, "f32")
    # cfg5: global sum + max over 2^30 f32 U[-1,1], seed 0
    def cfg5_global():
        return filled("f32", (1 << 30,), "uniform", 0, 0, -1.0, 1.0), T("f64", (1,)), T("f32", (1,))
    measure("cfg5_global_sum_max_f32", cfg5_global,
            lambda s: sdk.call("tensor_sum_max_f32", s[0], s[1], s[2]), 4_294_967_296, 1_073_741_824)
    return results


COPY_BYTES = 256 << 20  # calibration copy for counter runs: 256 MiB read + 256 MiB written


def pmc_probe(sdk, reps=3):
    """Workload for `rocprofv3 --pmc` runs: a plain 16-byte-vector copy of
    COPY_BYTES (known traffic, the calibration for FETCH_SIZE / WRITE_SIZE),
    then each cfg2 kernel, `reps` times each, with a 600 MB cache-flushing
    write between dispatches so that every dispatch starts from HBM."""
    from inference_c_amd import TensorView
    n = COPY_BYTES // 2
    src, dst = sdk.tensor("f16", (n,)), sdk.tensor("f16", (n,))
    flush = sdk.tensor("f32", (ROTATE_BYTES // 4,))
    sdk.call("tensor_fill_normal", src, 1, 9, 0.0, 1.0)
    t = {}
    t["x"], t["y"] = sdk.tensor("f16", (8192, 8192)), sdk.tensor("f16", (8192, 8192))
    t["a"], t["b"], t["o"] = (sdk.tensor("f16", (4096, 16384)) for _ in range(3))
    sdk.call("tensor_fill_normal", t["x"], 1, 0, 0.0, 1.0)
    sdk.call("tensor_fill_normal", t["a"], 1, 1, 0.0, 1.0)
    sdk.call("tensor_fill_normal", t["b"], 1, 2, 0.0, 1.0)
    view = TensorView.make((n,), (1,), 0)
    ops = [("copy_f16", lambda: sdk.call("tensor_view_add_mul_f16", src, view, None, None, dst)),
           ("silu_f16", lambda: sdk.call("tensor_silu_f16", t["x"], t["y"])),
           ("gelu_f16", lambda: sdk.call("tensor_gelu_f16", t["x"], t["y"])),
           ("swiglu_f16", lambda: sdk.call("tensor_silu_multiply_f16", t["b"], t["a"], t["o"]))]
    # the Q8_0 decode GEMV of the suite: [28672, 8192] packed weights, one row
    import numpy as np
    packed = np.random.default_rng(7).integers(0, 256, size=(28672, 256, 34), dtype=np.uint8)
    packed[:, :, 0:2] = np.frombuffer(np.float16(2.0 ** -7).tobytes(), np.uint8)
    t["w8"] = sdk.tensor("u8", packed.shape).upload(packed)
    t["x8"], t["y8"] = sdk.tensor("f16", (1, 8192)), sdk.tensor("f16", (1, 28672))
    sdk.call("tensor_fill_normal", t["x8"], 7, 3, 0.0, 1.0)
    del packed
    ops.append(("linear_q8_0_f16_1x8192_to_28672",
                lambda: sdk.call("tensor_linear_q8_0_f16", t["x8"], t["w8"], t["y8"])))
    # the configs[2..4] kernels at their BASELINE shapes
    t["x3"], t["y3"] = sdk.tensor("f16", (16384, 2048)), sdk.tensor("f16", (16384, 2048))
    t["w3"] = sdk.tensor("f16", (2048,))
    sdk.call("tensor_fill_normal", t["x3"], 3, 0, 0.0, 1.0)
    sdk.call("tensor_fill_uniform", t["w3"], 3, 1, 0.5, 1.5)
    ops.append(("cfg3_rms_norm_f16", lambda: sdk.call("tensor_rms_norm_f16", t["x3"], t["w3"],
                                                      1e-6, t["y3"])))
    t["lg"], t["sm"] = sdk.tensor("f16", (32, 2048, 2048)), sdk.tensor("f16", (32, 2048, 2048))
    t["rs"] = sdk.tensor("f32", (32, 2048))
    sdk.call("tensor_fill_normal", t["lg"], 3, 2, 0.0, 3.0)
    ops.append(("cfg3_causal_softmax_f16", lambda: sdk.call("tensor_softmax_f16", t["lg"], 1,
                                                            t["sm"])))
    ops.append(("cfg3_row_sum_f16", lambda: sdk.call("tensor_row_sum_f16", t["lg"], t["rs"])))
    ops.append(("cfg3_row_max_f16", lambda: sdk.call("tensor_row_max_f16", t["lg"], t["rs"])))
    B, S, H, D = 16, 1024, 32, 64
    perm = TensorView.make((B, H, S, D), (S * H * D, D, H * D, 1), 0)
    t["x4"], t["o4"] = sdk.tensor("f16", (B, S, H, D)), sdk.tensor("f16", (B, H, S, D))
    t["a4"], t["m4"] = sdk.tensor("f16", (1, H, 1, D)), sdk.tensor("f16", (B, 1, S, 1))
    sdk.call("tensor_fill_normal", t["x4"], 4, 0, 0.0, 1.0)
    sdk.call("tensor_fill_uniform", t["a4"], 4, 1, -1.0, 1.0)
    sdk.call("tensor_fill_uniform", t["m4"], 4, 2, -1.0, 1.0)
    ops.append(("cfg4_permuted_broadcast_f16", lambda: sdk.call(
        "tensor_view_add_mul_f16", t["x4"], perm, t["a4"], t["m4"], t["o4"])))
    t["x5"], t["r5"] = sdk.tensor("f16", (4096, 2048)), sdk.tensor("f16", (4096, 2048))
    t["h5"], t["n5"] = sdk.tensor("f16", (4096, 2048)), sdk.tensor("f16", (4096, 2048))
    sdk.call("tensor_fill_normal", t["x5"], 5, 0, 0.0, 1.0)
    sdk.call("tensor_fill_normal", t["r5"], 5, 1, 0.0, 1.0)
    ops.append(("cfg5_residual_rms_norm_f16", lambda: sdk.call(
        "tensor_residual_rms_norm_f16", t["x5"], t["r5"], t["w3"], 1e-6, t["h5"], t["n5"])))
    vocab, width, tokens = 32000, 2048, 32768
    t["emb"], t["eo"] = sdk.tensor("f16", (vocab, width)), sdk.tensor("f16", (tokens, width))
    sdk.call("tensor_fill_normal", t["emb"], 6, 0, 0.0, 1.0)
    t["ids"] = sdk.tensor("i32", (tokens,)).upload(
        ((np.arange(tokens, dtype=np.int64) * 2654435761) % vocab).astype(np.int32))
    ops.append(("embedding_lookup_f16", lambda: sdk.call("tensor_embedding_lookup_f16", t["emb"],
                                                         t["ids"], t["eo"])))
    # kernels that stage data in LDS, for the LDS instruction / bank-conflict
    # pass: RoPE (angle table), a [4096, 4096] f16 transpose (64x64 tiles),
    # the global sum/max (cross-wave combine) and flash attention f16 / f32
    t["q5"], t["k5"] = sdk.tensor("f16", (4096, 32, 64)), sdk.tensor("f16", (4096, 32, 64))
    sdk.call("tensor_fill_normal", t["q5"], 5, 2, 0.0, 1.0)
    sdk.call("tensor_fill_normal", t["k5"], 5, 3, 0.0, 1.0)
    ops.append(("rope_f16", lambda: sdk.call("tensor_rope_f16", t["q5"], t["k5"], 32, 32, 64,
                                             10000.0, 0)))
    t["xt"], t["yt"] = sdk.tensor("f16", (4096, 4096)), sdk.tensor("f16", (4096, 4096))
    sdk.call("tensor_fill_normal", t["xt"], 4, 0, 0.0, 1.0)
    transpose = TensorView.make((4096, 4096), (1, 4096), 0)
    ops.append(("transpose_f16", lambda: sdk.call("tensor_view_add_mul_f16", t["xt"], transpose,
                                                  None, None, t["yt"])))
    t["g"] = sdk.tensor("f32", (1 << 28,))
    t["gs"], t["gm"] = sdk.tensor("f64", (1,)), sdk.tensor("f32", (1,))
    sdk.call("tensor_fill_uniform", t["g"], 0, 5, -1.0, 1.0)
    ops.append(("global_sum_max_f32", lambda: sdk.call("tensor_sum_max_f32", t["g"], t["gs"],
                                                       t["gm"])))
    for dtype in ("f16", "f32"):
        qa = sdk.tensor(dtype, (1, 32, 2048, 128))
        ka, va = sdk.tensor(dtype, (1, 8, 2048, 128)), sdk.tensor(dtype, (1, 8, 2048, 128))
        oa = sdk.tensor(dtype, (1, 32, 2048, 128))
        for i, x in enumerate((qa, ka, va)):
            sdk.call("tensor_fill_normal", x, 6, i, 0.0, 1.0)
        t["attn_" + dtype] = (qa, ka, va, oa)
        ops.append((f"sdpa_{dtype}_prefill", lambda d=dtype: sdk.call(
            f"tensor_sdpa_device_{d}", *t["attn_" + d][:3], None, 0.08838834764831845, 1,
            t["attn_" + d][3])))
    for name, fn in ops:
        for _ in range(reps):
            sdk.call("tensor_fill_uniform", flush, 7, 0, -1.0, 1.0)
            fn()
            sdk.synchronize()
        print(f"pmc probe: {name} x{reps}", flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-suite", action="store_true", help="skip the per-config kernel suite")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only run the counter-collection workload (copy, cfg2 kernels and "
                         "the Q8_0 decode GEMV)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every GPU box here has one "
                          "GPU, and every op but the global reductions shards over rows or "
                          "tokens with no communication, so the one-GPU figure is the per-GPU "
                          "figure; run with --gpus 1"}))
        sys.exit(2)

    from inference_c_amd import Sdk
    sdk = Sdk()
    sdk.require_device()
    if args.pmc_probe:
        pmc_probe(sdk)
        return
    hip = Hip()
    stream = sdk.stream()

    # Each kernel gets its own rotation of identical operand sets, at least
    # 600 MB apart in traffic, so no launch finds its operands in the 256 MB
    # last-level cache.
    def filled(dtype, shape, stream_id):
        x = sdk.tensor(dtype, shape)
        sdk.call("tensor_fill_normal", x, 1, stream_id, 0.0, 1.0)
        return x

    def unary_sets():
        return [(filled("f16", (8192, 8192), 0), sdk.tensor("f16", (8192, 8192)))
                for _ in range(3)]

    silu_sets, gelu_sets = unary_sets(), unary_sets()
    swiglu_sets = [(filled("f16", (4096, 16384), 1), filled("f16", (4096, 16384), 2),
                    sdk.tensor("f16", (4096, 16384))) for _ in range(2)]
    sdk.synchronize()
    phases = [
        ("silu_f16", lambda i: sdk.call("tensor_silu_f16", *silu_sets[i % 3])),
        ("gelu_f16", lambda i: sdk.call("tensor_gelu_f16", *gelu_sets[i % 3])),
        # out = a * silu(b): b is the SiLU'd (gate) operand, a the up operand
        ("swiglu_f16", lambda i: sdk.call("tensor_silu_multiply_f16", swiglu_sets[i % 2][1],
                                          swiglu_sets[i % 2][0], swiglu_sets[i % 2][2])),
    ]
    for i in range(args.warmup):
        for _, fn in phases:
            fn(i)
    sdk.synchronize()
    # Timed region: K launches of each kernel, back to back on the SDK
    # stream, with one event before the first launch and one after each
    # kernel's K launches: per-kernel average = its phase / K.
    marks = [hip.event() for _ in range(len(phases) + 1)]
    t0 = time.perf_counter()
    hip.record(marks[0], stream)
    for j, (_, fn) in enumerate(phases):
        for i in range(args.steps):
            fn(i)
        hip.record(marks[j + 1], stream)
    sdk.synchronize()
    wall = time.perf_counter() - t0
    per_kernel = {name: hip.elapsed_ms(marks[j], marks[j + 1]) / args.steps
                  for j, (name, _) in enumerate(phases)}

    step_bytes = sum(v[0] for v in CFG2.values())
    step_elems = sum(v[1] for v in CFG2.values())
    ms_per_step = wall / args.steps * 1e3
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    dominant = max(per_kernel, key=per_kernel.get)
    achieved = CFG2[dominant][0] / (per_kernel[dominant] * 1e-3) / 1e9
    kernels = {name: {"avg_us": round(ms * 1e3, 2),
                      "gbps": round(CFG2[name][0] / (ms * 1e-3) / 1e9, 1),
                      "pct_peak": round(100 * CFG2[name][0] / (ms * 1e-3) / 1e9 / PEAK_GBPS, 1),
                      "elements_per_s": float(f"{CFG2[name][1] / (ms * 1e-3):.4g}")}
               for name, ms in per_kernel.items()}
    for group in (silu_sets, gelu_sets, swiglu_sets):
        for tensors in group:
            for v in tensors:
                v.free()

    line = {
        "metric": "achieved HBM GB/s and % of MI355X peak per tensor_ops kernel; elements/sec",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "BASELINE configs[1]: SiLU + tanh-GELU on [8192,8192] f16 N(0,1) "
                               "and SwiGLU a*silu(b) on [4096,16384] f16 N(0,1), seed 1, inputs "
                               "resident in HBM", "step_bytes": step_bytes,
                   "elements_per_step": step_elems},
        "pct_of_peak": round(100 * value / PEAK_GBPS, 1),
        "elements_per_s": float(f"{step_elems / (ms_per_step * 1e-3):.4g}"),
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1),
                     "peak": PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": measured_traffic(dominant),
                     "algorithmic_bytes": CFG2[dominant][0]},
        "kernels": kernels,
    }
    if not args.no_suite:
        line["suite"] = suite(sdk, hip, stream)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
