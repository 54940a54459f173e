#!/usr/bin/env python3
"""Benchmark of the BoaConstrictor batched compress/decompress hot path on one MI355X.

Workload (BASELINE.json configs[2] + configs[3]): d_model 256 x 8 Mamba layers, fp32, seeded random weights
(seed 0); 64 MiB of little-endian float32 records (per record 4 log-normal(mu=1, sigma=1.5) energies,
3 N(0,1) coordinates, 1 uniform int32 id; numpy default_rng(0)); chunks_count 4096 -> 4096 chunks of
16384 bytes.  One step = compress the whole payload (model parallel in time + fused range coding + device
compaction) and decompress it again (strictly sequential, one model step per byte), inputs resident in HBM.
value = input bytes / (compress time + decompress time), in MB/s (10^6 bytes/s).

Also reported: compress and decompress rates separately, the roofline of the dominant kernel from live HIP
event timing (boa_profile) inside the timed region, and a CPU baseline: this repo's restatement of the
reference CPU path (codec.compress_CPU / decompress_CPU: per-step torch-CPU model + per-lane range coding in
a thread pool) timed on a bounded sample of configs[0] on this host.
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
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_fused_step_d256x8L_4096lanes.json")

# rocprof names of the kernel instances each profiled class launches at the benchmark's shapes, default
# precision bf16x3 (k_gemm_bf<BM, BN, BK, EPI, NT, A split, C split>: EPI 0 none, 1 bias, 2 GELU, 4 residual)
KERNEL_NAMES = {
    ("compress", "gemm_in_proj"): "k_gemm_bf<128, 128, 32, 1, 3, true, false>",
    ("compress", "gemm_ff1"): "k_gemm_bf<128, 128, 32, 2, 3, true, true>",
    ("compress", "gemm_ff2"): "k_gemm_bf<128, 128, 32, 4, 3, true, false>",
    ("compress", "gemm_out_proj"): "k_gemm_bf<128, 128, 32, 1, 3, true, false>",
    ("compress", "gemm_x_proj"): "k_gemm_bf<64, 64, 128, 0, 3, false, false>",
    ("compress", "scan"): "k_scan<16, 16, true>",
    ("compress", "conv"): "k_conv_silu",
    ("decompress", "fused_step"): "k_fused_step<3>",
}


def fused_step_bytes(lanes: int, d: int = 256, L: int = 8, di: int = 512, ns: int = 16, V: int = 256) -> float:
    """Compulsory HBM bytes of one fused decode step (the library's own estimate, restated): SSM state read +
    write and conv history (3 reads + 1 write) per lane and layer, the input embedding row and coder state per
    lane, plus the bf16x3 weights (hi + lo) once."""
    params = L * (2 * di * d + (d // 16 + 2 * ns) * di + d * di + 4 * d * d * 2) + d * d + V * d
    return lanes * (L * (2.0 * di * ns * 4 + 4.0 * di * 4) + 4.0 * d + 64.0) + 4.0 * params


def measured_traffic(lanes: int, steps_per_launch: float):
    """HBM bytes per fused-step launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by the
    same counters on a copy kernel of known size), from the committed profile summary when it describes this
    launch shape; otherwise None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("lanes") != lanes:
        return None
    return t["bytes_per_step"] * steps_per_launch


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


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--payload-mib", type=int, default=64)
    ap.add_argument("--chunks", type=int, default=4096)
    ap.add_argument("--tile-len", type=int, default=int(os.environ.get("BOA_TILE_LEN", "64")))
    ap.add_argument("--cpu-steps", type=int, default=300, help="coded positions per chunk in the CPU sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 3 times (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (chunks are independent and would "
              "shard by range with one size exchange; see DESIGN.md)", file=sys.stderr)
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
    eng = M._Engine(W.seeded_blob(cfg, 0), cfg, B, args.tile_len)
    pitch = chunk + 8
    words = torch.empty((B, pitch), dtype=torch.int32, device=dev)
    nw = torch.empty(B, dtype=torch.int32, device=dev)
    offs = torch.empty(B, dtype=torch.int64, device=dev)
    payload = torch.empty(B * pitch, dtype=torch.int32, device=dev)
    out = torch.empty((B, chunk), dtype=torch.uint8, device=dev)
    stream = N.stream_ptr()
    log(f"[bench] context holds {eng.device_bytes / 2**30:.2f} GiB")

    def step():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        N.check(lib.boa_compress(eng.h, N.ptr(X), X.stride(0), N.ptr(lens), B, chunk, N.ptr(words), pitch,
                                 N.ptr(nw)))
        total = ctypes.c_int64(0)
        N.check(lib.boa_compact(N.ptr(words), pitch, N.ptr(nw), B, N.ptr(offs), N.ptr(payload), payload.numel(),
                                ctypes.byref(total), stream))
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        N.check(lib.boa_decompress(eng.h, N.ptr(payload), N.ptr(offs), N.ptr(nw), N.ptr(first), N.ptr(lens), B, chunk,
                                   N.ptr(out), out.stride(0)))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, total.value

    def read_profile():
        ents = (N.ProfEntry * 32)()
        n = ctypes.c_int32(0)
        N.check(lib.boa_profile_read(eng.h, ents, 32, ctypes.byref(n)))
        return {e.name.decode(): dict(launches=e.launches, sampled=e.sampled, ms=e.ms, flops=e.flops, bytes=e.bytes)
                for e in ents[:n.value]}

    for i in range(args.warmup):
        tc, td, tw = step()
        log(f"[bench] warmup {i}: compress {tc:.2f}s decompress {td:.2f}s words {tw}")
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
        pc = read_profile()
        N.check(lib.boa_profile(eng.h, 1))
        t1b = time.perf_counter()
        N.check(lib.boa_decompress(eng.h, N.ptr(payload), N.ptr(offs), N.ptr(nw), N.ptr(first), N.ptr(lens), B, chunk,
                                   N.ptr(out), out.stride(0)))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        pd = read_profile()
        N.check(lib.boa_profile(eng.h, 0))
        tcs.append(t1 - t0)
        tds.append(t2 - t1b)
        log(f"[bench] step {i}: compress {t1 - t0:.2f}s decompress {t2 - t1b:.2f}s words {total.value}")
        if i == 0:
            prof = {"compress": pc, "decompress": pd}
    ok = bool(torch.equal(out, X))
    comp_bytes = 4 * int(nw.sum().item())
    tc, td = float(np.mean(tcs)), float(np.mean(tds))

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
    if best is not None:
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
        roofline.update({"kernel": f"{phase}/{name}", "rocprof_name": KERNEL_NAMES.get((phase, name), name),
                         "avg_launch_ms": avg_ms, "algorithmic_per_launch": per_launch,
                         "launches": e["launches"], "time_share": best[0] / total_ms if total_ms else None})
        if name == "fused_step":
            roofline["steps_per_launch"] = round(per_launch / fused_step_bytes(B), 3)
            roofline["traffic"] = measured_traffic(B, roofline["steps_per_launch"])

    cpu = None
    if not args.no_cpu:
        log(f"[bench] CPU baseline: {args.cpu_steps} positions x 64 chunks")
        cpu = cpu_baseline(args.cpu_steps)
        log(f"[bench] CPU baseline {cpu['value']:.5f} MB/s in {cpu['seconds']:.1f}s")

    value = nbytes / (tc + td) / 1e6
    res = {
        "metric": METRIC,
        "value": value,
        "unit": "MB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": (tc + td) * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": ("configs[2]+configs[3]: compress then decompress 64 MiB float32 records (seed 0), "
                         f"{B} chunks x {chunk} B, d256x8L Mamba fp32 random init seed 0, inputs in HBM"),
            "chunks": B,
            "chunk_len": chunk,
            "payload_bytes": nbytes,
            "tile_len": args.tile_len,
        },
        "compress_MBps": nbytes / tc / 1e6,
        "decompress_MBps": nbytes / td / 1e6,
        "compress_MiBps": nbytes / tc / 2**20,
        "decompress_MiBps": nbytes / td / 2**20,
        "decompress_step_ms": td / (chunk - 1) * 1e3,
        "compressed_bytes": comp_bytes,
        "round_trip_ok": ok,
        "roofline": roofline,
        "kernel_ms": {k: round(v, 3) for k, v in sorted(share.items(), key=lambda kv: -kv[1])},
        "cpu_baseline": cpu,
    }
    if cpu:
        res["vs_cpu_compress"] = res["compress_MBps"] / cpu["compress_MBps"]
        res["vs_cpu_decompress"] = res["decompress_MBps"] / cpu["decompress_MBps"]
    print(json.dumps(res))


if __name__ == "__main__":
    main()
