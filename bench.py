#!/usr/bin/env python3
"""Benchmark of the BoaConstrictor batched compress/decompress hot path on one MI355X.

Workload (the benchmark's configs[2] + configs[3]): d_model 256 x 8 Mamba layers, fp32, seeded random weights
(seed 0); 64 MiB of little-endian float32 records (per record 4 log-normal(mu=1, sigma=1.5) energies,
3 N(0,1) coordinates, 1 uniform int32 id; numpy default_rng(0)); chunks_count 4096 -> 4096 chunks of
16384 bytes.  One step = compress the whole payload (model parallel in time + fused range coding + device
compaction) and decompress it again (strictly sequential, one model step per byte), inputs resident in HBM.
value = input bytes / (compress time + decompress time), in MB/s (10^6 bytes/s).

Arithmetic is the reference's: the default precision "f32" computes every GEMM in fp32 on the matrix cores
(v_mfma_f32_16x16x4_f32, fp32 operands and accumulation; the reference uses fp32 FMAs,
gemm_kernels.cu:168-280); LayerNorm, conv, scan, activations and the quantiser are fp32 / integer everywhere.
Warm-up steps are the same compress + decompress over the first --warmup-len bytes of every chunk (same
kernels, lanes and buffers; untimed), so that the driver's warm-up count does not multiply the run time.

Also reported: compress and decompress rates separately, the roofline of the dominant kernel from live HIP
event timing (boa_profile) inside the timed region, and a CPU baseline: this repo's restatement of the
reference CPU path (codec.compress_CPU / decompress_CPU: per-step torch-CPU model + per-lane range coding in
a thread pool) timed on a bounded sample of configs[0] on this host.  After the timed steps, untimed by the
headline, bounded extra measurements go into the same JSON line (--no-extras skips them):
  bf16x3_full_*  the same model and data at full size in the "bf16x3" mode (fp32 operands split into bf16
             hi + lo, three bf16 MFMA products per multiply-add, fp32 accumulation: ~16 significant bits per
             operand, narrower than the reference's fp32), one timed compress + decompress, with rooflines;
  coder      configs[1], the range coder alone: 16384 streams x 4096 symbols, P = 16;
  config4    configs[4]'s model (d512 x 16 layers, bf16 weights, seed 1) on its 16384 chunks of mixed
             int16/float32 records, each chunk cut to a stated length (steady-state rates);
  published_shape  (only with --published-shape) the shape of the reference's only published throughput
             (d256 x 1 layer, 4096-byte chunks; ~7 / ~5 MiB/s on an RTX 5090) in f32, on the headline's data.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "boa-constrictor_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "input MB/s compress + decompress, d256×8L Mamba, 4096 chunks, 1 GPU"
PEAK_BF16_MFMA_TFLOPS = 2500.0  # dense; a bf16x3 GEMM issues 3 bf16 products per model multiply-add
PEAK_HBM_GBPS = 8000.0
PEAK_F32_MFMA_TFLOPS = 157.3  # dense fp32 MFMA (v_mfma_f32_16x16x4_f32)
# measured HBM traffic of the fused decode kernel, per precision mode
TRAFFIC_FILES = {p: os.path.join(REPO, "profiles", f"traffic_fused_step_{p}_d256x8L_4096lanes.json")
                 for p in ("f32", "bf16x3")}
CODER_TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_rc_coder_configs1.json")

# rocprof names of the kernel instances each profiled class launches at the benchmark's shapes, per precision
# (k_gemm_bf<BM, BN, BK, EPI, NT, A split, C split>: EPI 0 none, 1 bias, 2 GELU, 4 residual; k_ffn<NT, true>:
# out_proj + LN2 + FF1 + GELU + FF2 + residual in one kernel; k_mixin<NT>: LN1 + in_proj + conv + x_proj;
# k_head_xq: head + quantiser; NT = 1 is the fp32 form, 3 the bf16x3 form)
KERNEL_NAMES = {
    "f32": {
        ("compress", "ffn"): "k_ffn<1, true>",
        ("compress", "mixin"): "k_mixin<1>",
        ("compress", "scan"): "k_scan<16, 16, false>",
        ("compress", "head_xq"): "k_head_xq<1, 256>",
        ("compress", "encode"): "k_encode_lf",
        ("decompress", "fused_step"): "k_fused_step<1, 512>",
    },
    "bf16x3": {
        ("compress", "gemm_in_proj"): "k_gemm_bf<128, 128, 32, 1, 3, true, false>",
        ("compress", "ffn"): "k_ffn<3, true>",
        ("compress", "mixin"): "k_mixin<3>",
        ("compress", "gemm_out_proj"): "k_gemm_bf<128, 128, 32, 1, 3, true, false>",
        ("compress", "gemm_x_proj"): "k_xproj<3, 3>",
        ("compress", "scan"): "k_scan<16, 16, true>",
        ("compress", "conv"): "k_conv_silu",
        ("compress", "head_xq"): "k_head_xq<3, 256>",
        ("compress", "encode"): "k_encode_lf",
        ("decompress", "fused_step"): "k_fused_step<3, 512>",
    },
}


def fused_step_bytes(lanes: int, d: int = 256, L: int = 8, di: int = 512, ns: int = 16, V: int = 256) -> float:
    """Compulsory HBM bytes of one fused decode step (the library's own estimate, restated): SSM state read +
    write and conv history (3 reads + 1 write) per lane and layer, the input embedding row and coder state per
    lane, plus the bf16x3 weights (hi + lo) once."""
    params = L * (2 * di * d + (d // 16 + 2 * ns) * di + d * di + 4 * d * d * 2) + d * d + V * d
    return lanes * (L * (2.0 * di * ns * 4 + 4.0 * di * 4) + 4.0 * d + 64.0) + 4.0 * params


def measured_traffic(lanes: int, steps_per_launch: float, precision: str):
    """HBM bytes per fused-step launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by the
    same counters on a copy kernel of known size), from the committed profile summary when it describes this
    launch shape and precision; otherwise None."""
    try:
        with open(TRAFFIC_FILES[precision]) as f:
            t = json.load(f)
    except (OSError, ValueError, KeyError):
        return None
    if t.get("lanes") != lanes:
        return None
    return t["bytes_per_step"] * steps_per_launch


def coder_traffic(streams: int, length: int):
    """The coder kernels' HBM bytes per launch measured with rocprofv3 --pmc (as measured_traffic), from the
    committed profile summary when it describes this workload; otherwise None."""
    try:
        with open(CODER_TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("streams") != streams or t.get("symbols_per_stream") != length:
        return None
    return t


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def synth_records(nbytes: int, seed: int = 0):
    """little-endian float32 records of 8 fields (32 B)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    n = nbytes // 32
    rec = np.empty((n, 8), dtype="<f4")
    rec[:, 0:4] = rng.lognormal(mean=1.0, sigma=1.5, size=(n, 4)).astype(np.float32)
    rec[:, 4:7] = rng.standard_normal((n, 3)).astype(np.float32)
    rec[:, 7] = rng.integers(-(1 << 31), 1 << 31, n, dtype=np.int64).astype(np.int32).view(np.float32)
    return rec.reshape(-1).view(np.uint8)


def markov_bytes(n: int, seed: int = 0, alpha: float = 0.1):
    """order-1 Markov chain over 256 symbols, Dirichlet(alpha) transition rows."""
    import numpy as np

    rng = np.random.default_rng(seed)
    P = rng.dirichlet([alpha] * 256, size=256)
    C = np.cumsum(P, axis=1)
    u = rng.random(n)
    out = np.empty(n, dtype=np.uint8)
    x = 0
    for i in range(n):
        out[i] = x
        x = min(int(np.searchsorted(C[x], u[i], side="right")), 255)
    return out


CODER_METRIC = "range coder alone: symbols/s encode + decode, 16384 streams x 4096 symbols, P=16, 1 GPU"


def coder_bench(args, steps: int, warmup: int, cpu_streams: int) -> dict:
    """per-step 256-symbol tables from N(0, 3^2) logits quantised to total 2^16 (min freq 1),
    symbols drawn from them, 16384 streams x 4096 symbols, generated on the device (not timed); then timed
    encodes and decodes over tables resident in HBM.  Byte-exact decode is checked on the device; the CPU
    leg runs this repo's C coder on the first cpu_streams streams and must produce the same words."""
    import numpy as np
    import torch

    from boa_amd import _native as N

    lib = N.lib()
    S, T, K, P = args.coder_streams, args.coder_len, 256, 16
    d_cdf = torch.empty((S, T, K), dtype=torch.int16, device="cuda")
    d_syms = torch.empty((S, T), dtype=torch.uint8, device="cuda")
    log(f"[coder] synthesising {S} x {T} tables ({d_cdf.numel() * 2 / 2**30:.1f} GiB)")
    N.check(lib.rc_synth_tables(0, 3.0, P, 2, K, S, T, N.ptr(d_cdf), N.ptr(d_syms), N.stream_ptr()))
    pitch = T + 8
    d_words = torch.zeros((S, pitch), dtype=torch.int32, device="cuda")
    d_n = torch.zeros(S, dtype=torch.int32, device="cuda")
    d_out = torch.zeros((S, T), dtype=torch.uint8, device="cuda")

    def enc():
        N.check(lib.rc_encode_tables(P, 2, N.ptr(d_cdf), K, N.ptr(d_syms), S, T, N.ptr(d_words), pitch, N.ptr(d_n),
                                     N.stream_ptr()))

    def dec():
        N.check(lib.rc_decode_tables(P, 2, N.ptr(d_cdf), K, N.ptr(d_words), pitch, N.ptr(d_n), S, T, N.ptr(d_out),
                                     N.stream_ptr()))

    for _ in range(warmup):
        enc()
        dec()
    te, td = [], []
    for _ in range(steps):
        e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        torch.cuda.synchronize()
        e0.record()
        enc()
        e1.record()
        dec()
        e2.record()
        torch.cuda.synchronize()
        te.append(e0.elapsed_time(e1) * 1e-3)
        td.append(e1.elapsed_time(e2) * 1e-3)
    ok = bool(torch.equal(d_out, d_syms))
    t_e, t_d = float(np.mean(te)), float(np.mean(td))
    nsym = S * T
    code_bytes = 4 * int(d_n.sum().item())
    # decode reads each step's full table row (K entries, 2 B) + writes 1 B; encode reads 2 entries + 1 B
    dec_bytes = nsym * (2.0 * K + 1) + code_bytes
    enc_bytes = nsym * (2.0 * 2 + 1) + code_bytes
    roofline = {"bound": "hbm", "kernel": "k_rc_decode_tables8<8>", "achieved": dec_bytes / t_d / 1e9,
                "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": dec_bytes / t_d / 1e9 / PEAK_HBM_GBPS, "traffic": None,
                "avg_launch_ms": t_d * 1e3, "algorithmic_per_launch": dec_bytes}
    measured = coder_traffic(S, T)
    encode_hbm = None
    if measured:
        roofline["traffic"] = measured["decode"]["bytes_per_launch"]
        # the encoder gathers 2 entries per symbol from a different row each: its HBM traffic is whole lines
        eb = measured["encode"]["bytes_per_launch"]
        encode_hbm = {"traffic": eb, "achieved": eb / t_e / 1e9, "unit": "GB/s", "frac": eb / t_e / 1e9 / PEAK_HBM_GBPS}
    cpu = None
    if not args.no_cpu:
        from oracle import ora

        ns = cpu_streams
        tab = d_cdf[:ns].cpu().numpy().view(np.uint16).astype(np.uint32)
        full = np.concatenate([tab, np.full((ns, T, 1), 1 << P, np.uint32)], axis=-1)
        syms = d_syms[:ns].cpu().numpy().astype(np.int32)
        words = d_words[:ns].cpu().numpy().view(np.uint32)
        nw = d_n[:ns].cpu().numpy()
        t0 = time.perf_counter()
        ref = [ora.encode_tables(P, full[i], syms[i]) for i in range(ns)]
        t1 = time.perf_counter()
        back = [ora.decode_tables(P, full[i], ref[i]) for i in range(ns)]
        t2 = time.perf_counter()
        same = all(np.array_equal(words[i, :nw[i]], ref[i]) for i in range(ns))
        rt = all(np.array_equal(back[i], syms[i]) for i in range(ns))
        cpu = {"value": ns * T / (t2 - t0), "unit": "symbols/s", "cores": 1, "kind": "port",
               "sample": f"first {ns} streams of the same tables (this repo's C coder, oracle/rc_oracle.c), "
                         "encode then decode, one thread",
               "encode_symbols_per_s": ns * T / (t1 - t0), "decode_symbols_per_s": ns * T / (t2 - t1),
               "words_identical_to_gpu": bool(same), "round_trip_ok": bool(rt)}
    res = {
        "metric": CODER_METRIC,
        "value": nsym / (t_e + t_d),
        "unit": "symbols/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": (t_e + t_d) * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic",
        "config": {"workload": f"configs[1]: {S} streams x {T} symbols, K=256, P=16, tables in HBM (int16 entries)",
                   "streams": S, "symbols_per_stream": T},
        "encode_symbols_per_s": nsym / t_e,
        "decode_symbols_per_s": nsym / t_d,
        "code_bytes": code_bytes,
        "round_trip_ok": ok,
        "roofline": roofline,
        "encode_hbm": encode_hbm,
        "cpu_baseline": cpu,
    }
    return res


def cpu_baseline(steps: int):
    import numpy as np
    import torch

    from boa_amd import weights as W
    from oracle import codec_ref, model_ref, weights_ref

    cores = len(os.sched_getaffinity(0))
    threads = min(cores, 16)
    torch.set_num_threads(threads)
    data = markov_bytes(1 << 20, seed=0)
    chunks = [data[i * 16384:(i + 1) * 16384] for i in range(64)]
    model = model_ref.RefModel(W.seeded_blob(W.Cfg(), 0), weights_ref.Cfg())
    t0 = time.perf_counter()
    words, fb, Ls, n_c = codec_ref.compress_cpu(model, chunks, num_workers=8, max_steps=steps)
    t1 = time.perf_counter()
    outs, n_d = codec_ref.decompress_cpu(model, words, [1 + n_c] * 64, fb, num_workers=8, max_steps=n_c)
    t2 = time.perf_counter()
    ok = all(np.array_equal(o[:1 + n_c], c[:1 + n_c]) for o, c in zip(outs, chunks))
    coded = 64 * n_c
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    c_mbps = coded / (t1 - t0) / 1e6
    d_mbps = coded / (t2 - t1) / 1e6
    return {
        "value": coded / ((t1 - t0) + (t2 - t1)) / 1e6,
        "unit": "MB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"configs[0] (1 MiB order-1 Markov, 64 chunks, d256x8L fp32 seed 0): first {n_c} coded "
                   f"positions of all 64 chunks, compress then decompress; torch threads {threads} of {cores} "
                   f"host cores, coder pool 8; {cpu_model}"),
        "compress_MBps": c_mbps,
        "decompress_MBps": d_mbps,
        "round_trip_ok": bool(ok),
        "seconds": t2 - t0,
    }


def lanes_equal(out, X, lens_h) -> bool:
    """Byte-exact round trip, lane by lane up to each lane's length (bytes past a lane's end are not
    written by the decoder and are not compared)."""
    import torch

    T = out.shape[1]
    L = torch.tensor(lens_h, dtype=torch.int64, device=out.device)
    mask = torch.arange(T, device=out.device)[None, :] < L[:, None]
    return bool(torch.equal(out[mask], X[:, :T][mask]))


def model_macs_per_token(d: int, L: int, V: int = 256, ns: int = 16) -> int:
    """GEMM multiply-adds per input byte: per layer in_proj, x_proj, dt_proj, out_proj, FF1, FF2; plus the
    two head layers."""
    di, r = 2 * d, -(-d // 16)
    per_layer = 2 * di * d + (r + 2 * ns) * di + r * di + d * di + 2 * 4 * d * d
    return L * per_layer + d * d + V * d


def decode_state_bytes(d: int, L: int, ns: int = 16) -> int:
    """Recurrent-state HBM bytes per decoded byte and lane: SSM state read + write and conv history (3 reads,
    1 write) of every layer."""
    di = 2 * d
    return L * (2 * di * ns * 4 + 4 * di * 4)


def codec_pass(lib, eng, X, lens, lens_h, chunk: int, reps: int, warm: int):
    """Untimed warm-ups, then `reps` timed compress (+ compaction) and decompress passes of X [B, chunk] on
    the context `eng`.  Returns mean compress and decompress seconds, compressed bytes, round-trip status."""
    import numpy as np
    import torch

    from boa_amd import _native as N

    B = X.shape[0]
    pitch = chunk + 8
    words = torch.empty((B, pitch), dtype=torch.int32, device="cuda")
    nw = torch.empty(B, dtype=torch.int32, device="cuda")
    offs = torch.empty(B, dtype=torch.int64, device="cuda")
    payload = torch.empty(B * pitch, dtype=torch.int32, device="cuda")
    out = torch.empty((B, chunk), dtype=torch.uint8, device="cuda")
    first = X[:, 0].contiguous()
    stream = N.stream_ptr()
    tcs, tds = [], []
    for i in range(warm + reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        N.check(lib.boa_compress(eng.h, N.ptr(X), X.stride(0), N.ptr(lens), B, chunk, N.ptr(words), pitch,
                                 N.ptr(nw)))
        total = ctypes.c_int64(0)
        N.check(lib.boa_compact(N.ptr(words), pitch, N.ptr(nw), B, N.ptr(offs), N.ptr(payload), payload.numel(),
                                ctypes.byref(total), stream))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        N.check(lib.boa_decompress(eng.h, N.ptr(payload), total.value, N.ptr(offs), N.ptr(nw), N.ptr(first),
                                   N.ptr(lens), B, chunk, N.ptr(out), out.stride(0)))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if i >= warm:
            tcs.append(t1 - t0)
            tds.append(t2 - t1)
    mean = lambda v: float(np.mean(v)) if v else 0.0
    return mean(tcs), mean(tds), 4 * int(nw.sum().item()), lanes_equal(out, X, lens_h)


def read_profile(lib, eng) -> dict:
    """Per-class event timings recorded by boa_profile since the window was opened."""
    from boa_amd import _native as N

    ents = (N.ProfEntry * 32)()
    n = ctypes.c_int32(0)
    N.check(lib.boa_profile_read(eng.h, ents, 32, ctypes.byref(n)))
    return {e.name.decode(): dict(launches=e.launches, sampled=e.sampled, ms=e.ms, flops=e.flops, bytes=e.bytes)
            for e in ents[:n.value]}


def fused_roofline(e: dict, B: int, precision: str) -> dict:
    """Roofline of the fused decode kernel from its boa_profile entry: model GEMM flops per launch against the
    MFMA peak of the precision's arithmetic (fp32 MFMA for f32; bf16 for bf16x3, counting its three products),
    and compulsory bytes per launch (SSM state read + write, conv history, embedding rows, coder state, the
    packed weights once per step) against HBM.  The binding one is the larger fraction."""
    avg_ms = e["ms"] / e["sampled"]
    per_launch_bytes = e["bytes"] / e["sampled"]
    steps = per_launch_bytes / fused_step_bytes(B)
    fpp = 2.0 * model_macs_per_token(256, 8)
    if precision == "f32":
        flops, peak = steps * B * fpp, PEAK_F32_MFMA_TFLOPS
    else:
        flops, peak = 3.0 * steps * B * fpp, PEAK_BF16_MFMA_TFLOPS
    t = avg_ms * 1e-3
    mfma = {"bound": "mfma", "achieved": flops / t / 1e12, "peak": peak, "unit": "TFLOP/s",
            "frac": flops / t / 1e12 / peak, "flops_per_launch": flops}
    hbm = {"bound": "hbm", "achieved": per_launch_bytes / t / 1e9, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
           "frac": per_launch_bytes / t / 1e9 / PEAK_HBM_GBPS, "bytes_per_launch": per_launch_bytes}
    return {"avg_launch_ms": avg_ms, "launches": e["launches"], "steps_per_launch": round(steps, 3), "mfma": mfma,
            "hbm": hbm}


def full_pass_extra(lib, X, lens_h, chunk: int, warm_len: int, precision: str) -> dict:
    """configs[2]+[3] at full size in another precision mode: the headline's model and data, one untimed warm-up
    pass on the first warm_len bytes of every chunk, then one timed compress (+ compaction) and decompress of
    the whole payload, with each kernel class's HIP events recorded (boa_profile) for the rooflines:
      compress    model GEMM flops (15,466,496 per coded position: every projection, dt_proj included,
                  = 2 x 7,733,248 multiply-adds; x3 for bf16x3's products) / compress time, against the MFMA
                  peak of the mode's arithmetic;
      decompress  the fused decode kernel's average launch (fused_roofline)."""
    import numpy as np  # noqa: F401
    import torch

    from boa_amd import _native as N
    from boa_amd import weights as W
    import model as M

    B = X.shape[0]
    cfg = W.Cfg()
    eng = M._Engine(W.seeded_blob(cfg, 0), cfg, B, 64, precision=precision)
    Xw = X[:, :warm_len].contiguous()
    lw = [min(warm_len, v) for v in lens_h]
    codec_pass(lib, eng, Xw, torch.tensor(lw, dtype=torch.int32, device="cuda"), lw, warm_len, reps=1, warm=0)
    lens = torch.tensor(lens_h, dtype=torch.int32, device="cuda")
    pitch = chunk + 8
    words = torch.empty((B, pitch), dtype=torch.int32, device="cuda")
    nw = torch.empty(B, dtype=torch.int32, device="cuda")
    offs = torch.empty(B, dtype=torch.int64, device="cuda")
    payload = torch.empty(B * pitch, dtype=torch.int32, device="cuda")
    out = torch.empty((B, chunk), dtype=torch.uint8, device="cuda")
    first = X[:, 0].contiguous()
    stream = N.stream_ptr()
    torch.cuda.synchronize()
    N.check(lib.boa_profile(eng.h, 1))
    t0 = time.perf_counter()
    N.check(lib.boa_compress(eng.h, N.ptr(X), X.stride(0), N.ptr(lens), B, chunk, N.ptr(words), pitch, N.ptr(nw)))
    total = ctypes.c_int64(0)
    N.check(lib.boa_compact(N.ptr(words), pitch, N.ptr(nw), B, N.ptr(offs), N.ptr(payload), payload.numel(),
                            ctypes.byref(total), stream))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    pc = read_profile(lib, eng)
    N.check(lib.boa_profile(eng.h, 1))
    t1b = time.perf_counter()
    N.check(lib.boa_decompress(eng.h, N.ptr(payload), total.value, N.ptr(offs), N.ptr(nw), N.ptr(first),
                               N.ptr(lens), B, chunk, N.ptr(out), out.stride(0)))
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    pd = read_profile(lib, eng)
    N.check(lib.boa_profile(eng.h, 0))
    ok = lanes_equal(out, X, lens_h)
    tc, td = t1 - t0, t2 - t1b
    nbytes = sum(lens_h)
    positions = sum(max(v - 1, 0) for v in lens_h)
    products = 1.0 if precision == "f32" else 3.0
    peak = PEAK_F32_MFMA_TFLOPS if precision == "f32" else PEAK_BF16_MFMA_TFLOPS
    fpp = 2.0 * model_macs_per_token(256, 8) * products
    p = f"{precision}_full_"
    res = {
        p + "workload": (f"configs[2]+configs[3] in {precision} mode: the headline's model and data, {B} chunks x "
                         f"{chunk} B, one warm-up pass on the first {warm_len} B of every chunk, then one timed "
                         "compress + decompress of the whole payload"),
        p + "compress_MBps": nbytes / tc / 1e6, p + "decompress_MBps": nbytes / td / 1e6,
        p + "MBps": nbytes / (tc + td) / 1e6,
        p + "decompress_step_ms": td / (chunk - 1) * 1e3,
        p + "compressed_bytes": 4 * int(total.value), p + "round_trip_ok": ok,
        p + "roofline_compress": {"bound": "mfma", "achieved": positions * fpp / tc / 1e12, "peak": peak,
                                  "unit": "TFLOP/s", "frac": positions * fpp / tc / 1e12 / peak,
                                  "flops_per_position": fpp, "positions": positions,
                                  "note": "whole compress pass (all kernels) against the MFMA peak"},
        p + "kernel_ms": {f"{ph}/{k}": round(e["ms"] * e["launches"] / e["sampled"], 3)
                          for ph, pp in (("compress", pc), ("decompress", pd)) for k, e in pp.items()
                          if e["sampled"]},
    }
    e = pd.get("fused_step")
    if e and e["sampled"]:
        res[p + "roofline_decompress"] = {"kernel": "decompress/fused_step",
                                          "rocprof_name": KERNEL_NAMES[precision][("decompress", "fused_step")],
                                          **fused_roofline(e, B, precision)}
    del eng, words, payload, offs, out
    torch.cuda.empty_cache()
    return res


def published_shape_extra(lib, X, lens_h, sub_len: int) -> dict:
    """The shape of the reference's only published throughput: ~7 "MB/s" (MiB/s, boa.cpp:39,404) compress and
    ~5 decompress on an NVIDIA RTX 5090 (portability_solved_cpp/README.md:66-68) for cms_experiment's model,
    d256 x 1 layer (experiments/cms_experiment/cms_experiment.yaml:10-11), chunks of 4096 B
    (portability_solved_cpp/README.md:45).  Here: d256 x 1 layer random init seed 0, the headline's chunks cut
    to their first sub_len bytes, in the reference's fp32 arithmetic ("f32" mode; the bf16x3 kernels are left to
    the headline, so that their profile averages describe it alone).  The CMS data and model are not shipped,
    so the inputs are the headline's synthetic records: an indication, not the same workload, and not
    `vs_baseline`."""
    import torch

    from boa_amd import weights as W
    import model as M

    B = X.shape[0]
    Xs = X[:, :sub_len].contiguous()
    ls = [min(sub_len, v) for v in lens_h]
    lens = torch.tensor(ls, dtype=torch.int32, device="cuda")
    nb = sum(ls)
    cfg = W.Cfg(n_layers=1)
    out = {"workload": (f"d256x1L random init seed 0, {B} chunks x first {sub_len} B of the headline's records; "
                        "one warm-up and one timed pass"),
           "published": {"compress_MiBps": 7.0, "decompress_MiBps": 5.0, "hardware": "NVIDIA RTX 5090",
                         "workload": "cms_experiment (CMS jets, not shipped), d256x1L, chunk 4096 B"}}
    for prec in ("f32",):
        eng = M._Engine(W.seeded_blob(cfg, 0), cfg, B, 64, precision=prec)
        tc, td, cb, ok = codec_pass(lib, eng, Xs, lens, ls, sub_len, reps=1, warm=1)
        del eng
        out[prec] = {"compress_MiBps": nb / tc / 2**20, "decompress_MiBps": nb / td / 2**20,
                     "compress_MBps": nb / tc / 1e6, "decompress_MBps": nb / td / 1e6,
                     "decompress_step_ms": td / (sub_len - 1) * 1e3, "round_trip_ok": ok}
        torch.cuda.empty_cache()
    return out


def config4_data(n_chunks: int, chunk: int, take: int, seed: int = 1):
    """configs[4] input: int16 N(0, 300^2) clipped to +-32767 and float32 log-normal(1, 1.5) records
    interleaved 1:1 (6-byte pairs), n_chunks x chunk bytes in all; returns the first `take` bytes of every
    chunk as an [n_chunks, take] uint8 array."""
    import numpy as np

    nbytes = n_chunks * chunk
    n = -(-nbytes // 6)
    rng = np.random.default_rng(seed)
    rec = np.empty(n, dtype=[("i", "<i2"), ("f", "<f4")])
    rec["i"] = np.clip(rng.normal(0.0, 300.0, n), -32767, 32767).astype(np.int16)
    rec["f"] = rng.lognormal(1.0, 1.5, n).astype(np.float32)
    flat = rec.view(np.uint8)[:nbytes].reshape(n_chunks, chunk)
    return np.ascontiguousarray(flat[:, :take])


def config4_extra(lib, lanes: int, take: int, wave: int = 0, warm_len: int = 0) -> dict:
    """d512 x 16 layers, bf16 weights (fp32 state, fp32 quantiser path), seed 1, `lanes` chunks
    of the 256 MiB mixed-record payload (chunks_count = lanes), each cut to its first `take` bytes (the whole
    chunk when take = 256 MiB / lanes), coded in waves of `wave` lanes (all of them by default) on one context;
    one untimed warm-up pass over the first `warm_len` bytes (default: take) of the first wave's chunks, then
    one timed compress + decompress per wave, summed.  Rooflines: compress against the dense bf16 MFMA peak
    with the model's multiply-adds (the bf16w mode issues two bf16 products per multiply-add: activation hi
    and lo parts), decompress against HBM with the recurrent state plus the bf16 weights once per step."""
    import numpy as np
    import torch

    from boa_amd import weights as W
    import model as M

    wave = wave or lanes
    warm_len = min(warm_len or take, take)
    if lanes % wave:
        raise ValueError(f"configs[4]: {lanes} chunks do not split into waves of {wave}")
    cfg = W.Cfg(d_model=512, n_layers=16)
    chunk = (256 << 20) // lanes
    data = config4_data(lanes, chunk, take)
    eng = M._Engine(W.seeded_blob(cfg, 1), cfg, wave, 64, precision="bf16w")
    lw = [warm_len] * wave
    Xw = torch.from_numpy(np.ascontiguousarray(data[:wave, :warm_len])).cuda()
    codec_pass(lib, eng, Xw, torch.tensor(lw, dtype=torch.int32, device="cuda"), lw, warm_len, reps=0, warm=1)
    del Xw
    ls = [take] * wave
    lens = torch.tensor(ls, dtype=torch.int32, device="cuda")
    tc = td = 0.0
    cb, ok = 0, True
    for w in range(lanes // wave):
        X = torch.from_numpy(np.ascontiguousarray(data[w * wave:(w + 1) * wave])).cuda()
        tcw, tdw, cbw, okw = codec_pass(lib, eng, X, lens, ls, take, reps=1, warm=0)
        if lanes != wave:
            log(f"[bench] configs[4] wave {w}: compress {tcw:.2f}s decompress {tdw:.2f}s round trip {okw}")
        tc, td, cb, ok = tc + tcw, td + tdw, cb + cbw, ok and okw
        del X
    del eng
    nb = lanes * take
    macs = model_macs_per_token(512, 16)
    flops = 2.0 * macs * lanes * (take - 1)
    step_s = td / (take - 1)
    step_bytes = lanes * decode_state_bytes(512, 16) + 2.0 * macs
    return {
        "workload": (f"configs[4]: d512x16L bf16 weights seed 1, {lanes} chunks of the 256 MiB int16/float32 "
                     f"record payload, first {take} B of each chunk, in waves of {wave} lanes; one warm-up pass "
                     f"over the first {warm_len} B, then one timed pass"),
        "compress_MBps": nb / tc / 1e6, "decompress_MBps": nb / td / 1e6, "decompress_step_ms": step_s * 1e3,
        "compressed_bytes": cb, "round_trip_ok": ok,
        "roofline_compress": {"bound": "mfma", "achieved": flops / tc / 1e12, "peak": PEAK_BF16_MFMA_TFLOPS,
                              "unit": "TFLOP/s", "frac": flops / tc / 1e12 / PEAK_BF16_MFMA_TFLOPS,
                              "flops_per_byte": 2 * macs},
        "roofline_decompress": {"bound": "hbm", "achieved": step_bytes / step_s / 1e9, "peak": PEAK_HBM_GBPS,
                                "unit": "GB/s", "frac": step_bytes / step_s / 1e9 / PEAK_HBM_GBPS,
                                "bytes_per_step": step_bytes},
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--payload-mib", type=int, default=64)
    ap.add_argument("--chunks", type=int, default=4096)
    ap.add_argument("--tile-len", type=int, default=int(os.environ.get("BOA_TILE_LEN", "64")))
    ap.add_argument("--cpu-steps", type=int, default=500, help="coded positions per chunk in the CPU sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", choices=["codec", "coder", "config4"], default="codec",
                    help="codec: configs[2]+[3] (the metric); coder: configs[1], the range coder alone; config4: "
                         "configs[4] alone (the bounded run the default line carries as its config4 extra)")
    ap.add_argument("--coder-streams", type=int, default=16384)
    ap.add_argument("--coder-len", type=int, default=4096)
    ap.add_argument("--coder-cpu-streams", type=int, default=64)
    ap.add_argument("--precision", choices=["f32", "bf16x3"], default="f32",
                    help="GEMM arithmetic of the headline: f32 (fp32 MFMA, the reference's arithmetic) or bf16x3")
    ap.add_argument("--warmup-len", type=int, default=1024,
                    help="bytes per chunk of each untimed warm-up step (the same kernels over a prefix)")
    ap.add_argument("--no-extras", action="store_true", help="skip the bf16x3, coder and configs[4] extras")
    ap.add_argument("--alt-warm-len", type=int, default=256,
                    help="bytes per chunk of the untimed warm-up before the full-size bf16x3 pass")
    ap.add_argument("--no-alt-full", action="store_true", help="skip the full-size bf16x3 pass")
    ap.add_argument("--published-shape", action="store_true",
                    help="also run the published-shape extra (d256x1L in f32 mode; off by default, so that the "
                         "f32 kernels' profile averages describe the 8-layer model alone)")
    ap.add_argument("--pub-len", type=int, default=4096,
                    help="bytes per chunk of the published-shape extra (d256x1L; the reference's chunk size)")
    ap.add_argument("--c4-lanes", type=int, default=16384, help="chunks (= lanes) of the configs[4] extra")
    ap.add_argument("--c4-len", type=int, default=257,
                    help="bytes per chunk of the configs[4] extra (257: 256 coded positions, four whole tiles)")
    ap.add_argument("--c4-wave", type=int, default=0,
                    help="lanes per wave of the configs[4] run (default: all chunks in one wave)")
    ap.add_argument("--c4-warm-len", type=int, default=0,
                    help="bytes per chunk of the configs[4] warm-up pass (default: --c4-len)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 3 times (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (chunks are independent and would "
              "shard by contiguous chunk range with one exchange of payload sizes)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from boa_amd import _native as N
    from boa_amd import weights as W
    import model as M

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                          "launches": 3}))
        return
    if args.workload == "coder":
        print(json.dumps(coder_bench(args, args.steps, args.warmup, args.coder_cpu_streams)))
        return
    if args.workload == "config4":
        print(json.dumps({"metric": "configs[4] input MB/s compress, decompress, d512x16L bf16 weights, 1 GPU",
                          **config4_extra(N.lib(), args.c4_lanes, args.c4_len, args.c4_wave, args.c4_warm_len)}))
        return
    lib = N.lib()
    dev = torch.device("cuda")
    nbytes = args.payload_mib << 20
    B = args.chunks
    chunk = -(-nbytes // B)
    log(f"[bench] synthesising {nbytes} bytes, {B} chunks of {chunk}")
    data = synth_records(nbytes, 0)
    host = torch.zeros((B, chunk), dtype=torch.uint8, pin_memory=True)
    host.view(-1)[:nbytes] = torch.from_numpy(data)
    lens_h = [min(chunk, nbytes - i * chunk) for i in range(B)]
    X = host.to(dev)
    lens = torch.tensor(lens_h, dtype=torch.int32, device=dev)
    first = X[:, 0].contiguous()
    cfg = W.Cfg()
    prec = args.precision
    eng = M._Engine(W.seeded_blob(cfg, 0), cfg, B, args.tile_len, precision=prec)
    pitch = chunk + 8
    words = torch.empty((B, pitch), dtype=torch.int32, device=dev)
    nw = torch.empty(B, dtype=torch.int32, device=dev)
    offs = torch.empty(B, dtype=torch.int64, device=dev)
    payload = torch.empty(B * pitch, dtype=torch.int32, device=dev)
    out = torch.empty((B, chunk), dtype=torch.uint8, device=dev)
    stream = N.stream_ptr()
    log(f"[bench] context holds {eng.device_bytes / 2**30:.2f} GiB")

    # warm-up step: the same calls over the first wl bytes of every chunk (X keeps its row stride)
    wl = max(2, min(args.warmup_len, chunk))
    lens_w = torch.clamp(lens, max=wl)

    def warm_step():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        N.check(lib.boa_compress(eng.h, N.ptr(X), X.stride(0), N.ptr(lens_w), B, wl, N.ptr(words), pitch,
                                 N.ptr(nw)))
        total = ctypes.c_int64(0)
        N.check(lib.boa_compact(N.ptr(words), pitch, N.ptr(nw), B, N.ptr(offs), N.ptr(payload), payload.numel(),
                                ctypes.byref(total), stream))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        N.check(lib.boa_decompress(eng.h, N.ptr(payload), total.value, N.ptr(offs), N.ptr(nw), N.ptr(first),
                                   N.ptr(lens_w), B, wl, N.ptr(out), out.stride(0)))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, total.value

    for i in range(args.warmup):
        tc, td, tw = warm_step()
        log(f"[bench] warmup {i} ({wl} B per chunk): compress {tc:.2f}s decompress {td:.2f}s words {tw}")
    tcs, tds = [], []
    prof = {"compress": {}, "decompress": {}}
    for i in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        N.check(lib.boa_profile(eng.h, 1))
        N.check(lib.boa_compress(eng.h, N.ptr(X), X.stride(0), N.ptr(lens), B, chunk, N.ptr(words), pitch, N.ptr(nw)))
        total = ctypes.c_int64(0)
        N.check(lib.boa_compact(N.ptr(words), pitch, N.ptr(nw), B, N.ptr(offs), N.ptr(payload), payload.numel(),
                                ctypes.byref(total), stream))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        pc = read_profile(lib, eng)
        N.check(lib.boa_profile(eng.h, 1))
        t1b = time.perf_counter()
        N.check(lib.boa_decompress(eng.h, N.ptr(payload), total.value, N.ptr(offs), N.ptr(nw), N.ptr(first),
                                   N.ptr(lens), B, chunk, N.ptr(out), out.stride(0)))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        pd = read_profile(lib, eng)
        N.check(lib.boa_profile(eng.h, 0))
        tcs.append(t1 - t0)
        tds.append(t2 - t1b)
        log(f"[bench] step {i}: compress {t1 - t0:.2f}s decompress {t2 - t1b:.2f}s words {total.value}")
        if i == 0:
            prof = {"compress": pc, "decompress": pd}
    ok = lanes_equal(out, X, lens_h)
    comp_bytes = 4 * int(nw.sum().item())
    tc, td = float(np.mean(tcs)), float(np.mean(tds))
    # PCIe legs of the host-memory API (codec.compress_GPU / decompress_GPU): input H2D + payload D2H for
    # compress, payload H2D + output D2H for decompress, pinned host buffers, timed on their own
    host_payload = torch.empty(comp_bytes // 4, dtype=torch.int32, pin_memory=True)
    host_out = torch.empty_like(host, pin_memory=True)

    def timed(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t

    t_h2d_in = timed(lambda: X.copy_(host, non_blocking=True))
    t_d2h_pl = timed(lambda: host_payload.copy_(payload[:comp_bytes // 4], non_blocking=True))
    t_h2d_pl = timed(lambda: payload[:comp_bytes // 4].copy_(host_payload, non_blocking=True))
    t_d2h_out = timed(lambda: host_out.copy_(out, non_blocking=True))

    # dominant kernel: largest estimated total time (sampled time scaled to all launches)
    share = {}
    best = None
    for phase, pp in prof.items():
        for name, e in pp.items():
            if e["sampled"] == 0:
                continue
            tot_ms = e["ms"] * e["launches"] / e["sampled"]
            share[f"{phase}/{name}"] = tot_ms
            if best is None or tot_ms > best[0]:
                best = (tot_ms, phase, name, e)
    total_ms = sum(share.values())
    roofline = None
    if best is not None and best[2] == "fused_step":
        _, phase, name, e = best
        fr = fused_roofline(e, B, prec)
        # the binding resource: fp32 MFMA for the f32 form (its GEMM phases), HBM for the split forms
        main = fr["mfma"] if fr["mfma"]["frac"] >= fr["hbm"]["frac"] else fr["hbm"]
        roofline = {k: main[k] for k in ("bound", "achieved", "peak", "unit", "frac")}
        roofline["traffic"] = measured_traffic(B, fr["steps_per_launch"], prec)
        roofline.update({"kernel": f"{phase}/{name}", "rocprof_name": KERNEL_NAMES[prec].get((phase, name), name),
                         "avg_launch_ms": fr["avg_launch_ms"], "launches": fr["launches"],
                         "steps_per_launch": fr["steps_per_launch"],
                         "algorithmic_per_launch": main.get("flops_per_launch", main.get("bytes_per_launch")),
                         "time_share": best[0] / total_ms if total_ms else None,
                         "other_bound": fr["hbm"] if main is fr["mfma"] else fr["mfma"]})
    elif best is not None:
        _, phase, name, e = best
        avg_ms = e["ms"] / e["sampled"]
        if name.startswith("gemm"):
            achieved = 3.0 * e["flops"] / (e["ms"] * 1e-3) / 1e12  # bf16 MFMA flops (3 products)
            roofline = {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_MFMA_TFLOPS, "unit": "TFLOP/s",
                        "frac": achieved / PEAK_BF16_MFMA_TFLOPS, "traffic": None}
            per_launch = 3.0 * e["flops"] / e["sampled"]
        else:
            achieved = e["bytes"] / (e["ms"] * 1e-3) / 1e9
            roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                        "frac": achieved / PEAK_HBM_GBPS, "traffic": None}
            per_launch = e["bytes"] / e["sampled"]
        roofline.update({"kernel": f"{phase}/{name}", "rocprof_name": KERNEL_NAMES[prec].get((phase, name), name),
                         "avg_launch_ms": avg_ms, "algorithmic_per_launch": per_launch,
                         "launches": e["launches"], "time_share": best[0] / total_ms if total_ms else None})

    cpu = None
    if not args.no_cpu:
        log(f"[bench] CPU baseline: {args.cpu_steps} positions x 64 chunks")
        cpu = cpu_baseline(args.cpu_steps)
        log(f"[bench] CPU baseline {cpu['value']:.5f} MB/s in {cpu['seconds']:.1f}s")

    extras = {}
    if not args.no_extras:
        del words, payload, offs, eng
        torch.cuda.empty_cache()
        alt = "bf16x3" if prec == "f32" else "f32"
        if not args.no_alt_full:
            log(f"[bench] extra: {alt} mode, full size ({B} chunks x {chunk} B)")
            extras.update(full_pass_extra(lib, X, lens_h, chunk, args.alt_warm_len, alt))
            log(f"[bench] extra: {alt} compress {extras[alt + '_full_compress_MBps']:.3f} MB/s, decompress "
                f"{extras[alt + '_full_decompress_MBps']:.3f} MB/s "
                f"({extras[alt + '_full_decompress_step_ms']:.3f} ms per step), round trip "
                f"{extras[alt + '_full_round_trip_ok']}")
        if args.published_shape:
            log(f"[bench] extra: the published shape (d256x1L, first {args.pub_len} B of each chunk)")
            extras["published_shape"] = published_shape_extra(lib, X, lens_h, args.pub_len)
            log(f"[bench] extra: d256x1L f32 compress "
                f"{extras['published_shape']['f32']['compress_MiBps']:.2f} MiB/s, decompress "
                f"{extras['published_shape']['f32']['decompress_MiBps']:.2f} MiB/s")
        log("[bench] extra: range coder alone (configs[1])")
        extras["coder"] = coder_bench(args, 3, 1, args.coder_cpu_streams if not args.no_cpu else 0)
        log(f"[bench] extra: coder {extras['coder']['value'] / 1e9:.2f} G symbols/s, round trip "
            f"{extras['coder']['round_trip_ok']}")
        torch.cuda.empty_cache()
        log(f"[bench] extra: configs[4] on {args.c4_lanes} chunks x {args.c4_len} B")
        extras["config4"] = config4_extra(lib, args.c4_lanes, args.c4_len)
        log(f"[bench] extra: configs[4] compress {extras['config4']['compress_MBps']:.3f} MB/s, decompress "
            f"{extras['config4']['decompress_MBps']:.3f} MB/s, round trip {extras['config4']['round_trip_ok']}")

    value = nbytes / (tc + td) / 1e6
    positions = sum(max(v - 1, 0) for v in lens_h)
    c_fpp = 2.0 * model_macs_per_token(256, 8) * (1.0 if prec == "f32" else 3.0)
    c_peak = PEAK_F32_MFMA_TFLOPS if prec == "f32" else PEAK_BF16_MFMA_TFLOPS
    res = {
        "metric": METRIC,
        "value": value if ok else None,
        "unit": "MB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": (tc + td) * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if prec == "f32" else "bf16x3",
        "data": "synthetic",
        "config": {
            "workload": ("configs[2]+configs[3]: compress then decompress 64 MiB float32 records (seed 0), "
                         f"{B} chunks x {chunk} B, d256x8L Mamba random init seed 0 (fp32 weights), GEMMs in "
                         + ("fp32 on the matrix cores (v_mfma_f32_16x16x4_f32, fp32 operands and accumulation)"
                            if prec == "f32" else
                            "bf16x3 (fp32 operands split into bf16 hi+lo, three bf16 MFMA products, fp32 "
                            "accumulation)")
                         + f", inputs in HBM; warm-up steps over the first {wl} B of every chunk"),
            "chunks": B,
            "chunk_len": chunk,
            "payload_bytes": nbytes,
            "tile_len": args.tile_len,
            "precision": prec,
            "warmup_len": wl,
        },
        "compress_MBps": nbytes / tc / 1e6,
        "decompress_MBps": nbytes / td / 1e6,
        "compress_MiBps": nbytes / tc / 2**20,
        "decompress_MiBps": nbytes / td / 2**20,
        "decompress_step_ms": td / (chunk - 1) * 1e3,
        "compressed_bytes": comp_bytes,
        "host_compress_MBps": nbytes / (tc + t_h2d_in + t_d2h_pl) / 1e6,
        "host_decompress_MBps": nbytes / (td + t_h2d_pl + t_d2h_out) / 1e6,
        "pcie_ms": {"input_h2d": t_h2d_in * 1e3, "payload_d2h": t_d2h_pl * 1e3, "payload_h2d": t_h2d_pl * 1e3,
                    "output_d2h": t_d2h_out * 1e3},
        "round_trip_ok": ok,
        "roofline": roofline,
        "roofline_compress": {"bound": "mfma", "achieved": positions * c_fpp / tc / 1e12, "peak": c_peak,
                              "unit": "TFLOP/s", "frac": positions * c_fpp / tc / 1e12 / c_peak,
                              "flops_per_position": c_fpp, "positions": positions,
                              "note": "whole compress pass (all kernels) against the MFMA peak of the mode"},
        "kernel_ms": {k: round(v, 3) for k, v in sorted(share.items(), key=lambda kv: -kv[1])},
        "cpu_baseline": cpu,
    }
    if cpu:
        res["vs_cpu_compress"] = res["compress_MBps"] / cpu["compress_MBps"]
        res["vs_cpu_decompress"] = res["decompress_MBps"] / cpu["decompress_MBps"]
    res.update(extras)
    print(json.dumps(res))
    if not ok:
        log("[bench] round trip FAILED: the headline value is withheld")
        sys.exit(1)


if __name__ == "__main__":
    main()
