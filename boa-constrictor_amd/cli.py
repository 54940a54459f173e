"""Command line for the compress / decompress path, with the reference CLI's flags and config keys.

Reference: main.py:54-70 (flags) and main.py:140-260, 440-540 (config keys, output names, compress /
decompress / verify flow).  Only the hot path is provided: compress a file into ``<name>.boa``, decompress it
into ``<name>_decompressed.<ext>``, verify, print timings.  Training, evaluation, baseline comparisons and the
interactive experiment creator are not part of this build and are rejected with an error.

    python cli.py --config exp.yaml [--compress-only | --decompress-only] [--verify] [--show-timings]
                  [--model-path model.pt|model.bin] [--no-progress] [--precision fp32|bf16x3|f32|bf16w]

Config keys read (as main.py reads them): ``name`` (default: the config file's stem), ``experiments_root``
(default ``experiments``), ``model.d_model``, ``model.num_layers``, ``model.vocab_size``, ``model_path`` or
``model.path``, ``compression.file_to_compress`` (or top-level ``file_path``), ``compression.chunks_count``
(default 1000, main.py:485), ``verify``, ``progress``, ``precision``.  Without a model path the model is a
seeded random init (``model.seed``, default 0): the reference would train one first.
"""
from __future__ import annotations

import argparse
import os
import sys
import time
from pathlib import Path
from typing import Dict, List, Optional

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

# The reference's --precision choices (main.py:59) map onto this build's GEMM arithmetic: "fp32" is plain
# float32 arithmetic (fp32 MFMA, the "f32" mode), as the reference computes it.  The build's own mode names
# are accepted as well: "bf16x3" (fp32 operands split into bfloat16 hi + lo, three products, fp32
# accumulation; faster, about 16 significant bits per operand) and "bf16w" (bfloat16 weights).  The
# reference's "fp16" / "fp8" choices select training precisions that this build does not have.
PRECISION_MAP = {"fp32": "f32", "f32": "f32", "bf16x3": "bf16x3", "bf16w": "bf16w"}
UNSUPPORTED_FLAGS = ("new_experiment", "train_only", "evaluate", "evaluate_only", "comparison_baseline_only")


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="BoaConstrictor compress / decompress (MI355X build)")
    p.add_argument("--config", "-c", type=Path, required=True, help="Path to YAML experiment config")
    p.add_argument("--no-progress", action="store_true", help="Disable progress bars")
    p.add_argument("--device", type=str, default="cuda", help="cuda (the ROCm GPU); cpu is not supported")
    p.add_argument("--precision", type=str, default=None, choices=sorted(PRECISION_MAP), help="GEMM arithmetic")
    p.add_argument("--compress-only", action="store_true", help="Only run compression")
    p.add_argument("--decompress-only", action="store_true", help="Only run decompression")
    p.add_argument("--show-timings", action="store_true", help="Print timings for each major operation")
    p.add_argument("--verify", action="store_true", help="After decompression, verify bytes match the input file")
    p.add_argument("--model-path", type=str, default=None, help="Model .pt (state_dict) or converted .bin")
    for flag in UNSUPPORTED_FLAGS:
        p.add_argument("--" + flag.replace("_", "-"), action="store_true", help=argparse.SUPPRESS)
    return p.parse_args(argv)


def load_config(path: Path) -> Dict:
    import yaml

    with open(path) as f:
        cfg = yaml.safe_load(f) or {}
    if not isinstance(cfg, dict):
        raise ValueError(f"{path}: the config must be a mapping")
    return cfg


def resolve(args: argparse.Namespace, cfg: Dict) -> Dict:
    """Paths and settings as main.py derives them (relative paths are relative to the config's directory)."""
    for flag in UNSUPPORTED_FLAGS:
        if getattr(args, flag):
            raise SystemExit(f"--{flag.replace('_', '-')} is not part of this build (compress/decompress only)")
    if args.device != "cuda":
        raise SystemExit("only --device cuda (the ROCm GPU) is supported")
    cfg_dir = args.config.resolve().parent
    name = cfg.get("name") or args.config.stem
    model = cfg.get("model", {}) or {}
    comp = cfg.get("compression", {}) or {}

    def rel(p: Optional[str]) -> Optional[Path]:
        if not p:
            return None
        q = Path(p).expanduser()
        return q if q.is_absolute() else (cfg_dir / q).resolve()

    model_path = Path(args.model_path).expanduser() if args.model_path else rel(cfg.get("model_path") or model.get("path"))
    src = rel(comp.get("file_to_compress") or cfg.get("file_path"))
    root = rel(cfg.get("experiments_root", "experiments"))
    exp_dir = root / name
    precision = args.precision or str(cfg.get("precision", "fp32"))
    if precision not in PRECISION_MAP:
        raise SystemExit(f"precision {precision!r} is not supported here (choose from {sorted(PRECISION_MAP)})")
    return {
        "name": name,
        "exp_dir": exp_dir,
        "boa_path": exp_dir / f"{name}.boa",
        "src": src,
        "model_path": model_path,
        "d_model": int(model.get("d_model", 256)),
        "num_layers": int(model.get("num_layers", 8)),
        "vocab_size": int(model.get("vocab_size", 256)),
        "seed": int(model.get("seed", 0)),
        "chunks_count": int(comp.get("chunks_count", 1000)),
        "precision": PRECISION_MAP[precision],
        "verify": bool(args.verify or cfg.get("verify", False)),
        "progress": (not args.no_progress) and bool(cfg.get("progress", True)),
    }


def build_model(r: Dict):
    import torch

    from boa_amd import weights as W
    import model as M

    mp = r["model_path"]
    if mp is not None and mp.suffix == ".bin":
        cfg = W.Cfg(d_model=r["d_model"], n_layers=r["num_layers"], vocab=r["vocab_size"])
        m = M.BoaConstrictor(cfg.d_model, cfg.n_layers, cfg.vocab).load_blob(W.read_bin(str(mp), cfg))
    elif mp is not None:
        sd = torch.load(str(mp), map_location="cpu", weights_only=True)
        if isinstance(sd, dict) and "model_state_dict" in sd:
            sd = sd["model_state_dict"]
        cfg = W.infer_cfg(sd)
        m = M.BoaConstrictor(cfg.d_model, cfg.n_layers, cfg.vocab)
        m.load_state_dict(sd, strict=True)
    else:
        cfg = W.Cfg(d_model=r["d_model"], n_layers=r["num_layers"], vocab=r["vocab_size"])
        m = M.BoaConstrictor(cfg.d_model, cfg.n_layers, cfg.vocab).load_blob(W.seeded_blob(cfg, r["seed"]))
    m.precision = r["precision"]
    return m


def main(argv: Optional[List[str]] = None) -> int:
    args = parse_args(argv)
    r = resolve(args, load_config(args.config))
    import torch  # noqa: F401  (before the HIP library is loaded)

    import boa

    if args.compress_only and args.decompress_only:
        raise SystemExit("--compress-only and --decompress-only exclude each other")
    r["exp_dir"].mkdir(parents=True, exist_ok=True)
    timings: Dict[str, float] = {}
    t0 = time.perf_counter()
    model = build_model(r)
    timings["model"] = time.perf_counter() - t0
    f = boa.BOA("cuda", str(r["boa_path"]), model)
    ok = True
    if not args.decompress_only:
        if r["src"] is None or not r["src"].exists():
            raise SystemExit(f"compression input not found: {r['src']}")
        print("Starting compression...")
        t0 = time.perf_counter()
        f.compress(str(r["src"]), chunks_count=r["chunks_count"], progress=r["progress"])
        timings["compression"] = time.perf_counter() - t0
        size_in, size_out = r["src"].stat().st_size, r["boa_path"].stat().st_size
        print(f"Compression ratio: {size_in / size_out if size_out else float('inf'):.2f}")
        print(f"Compression complete in {timings['compression']:.2f}s")
    if not args.compress_only:
        print("Starting decompression...")
        t0 = time.perf_counter()
        data = boa.BOA("cuda", str(r["boa_path"]), model).decompress(progress=r["progress"])
        ext = (r["src"].suffix.lstrip(".") if r["src"] is not None else "") or "bin"
        out_path = r["exp_dir"] / f"{r['name']}_decompressed.{ext}"
        with open(out_path, "wb") as fo:
            fo.write(data)
        timings["decompression"] = time.perf_counter() - t0
        print(f"Decompression complete in {timings['decompression']:.2f}s")
        if r["verify"]:
            ref = r["src"].read_bytes() if r["src"] is not None else b""
            if data == ref:
                print(f"VERIFY: OK — decompressed output matches input ({len(data)} bytes)")
            else:
                ok = False
                print("VERIFY: MISMATCH — decompressed output differs from input")
                if len(data) != len(ref):
                    print(f"  Sizes differ: decompressed={len(data)} vs input={len(ref)}")
                else:
                    i = next(i for i in range(len(data)) if data[i] != ref[i])
                    print(f"  First differing byte at offset {i}: dec={data[i]} input={ref[i]}")
    if args.show_timings:
        for k, v in timings.items():
            print(f"  {k}: {v:.3f}s")
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
