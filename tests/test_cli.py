"""cli.py: flags and config keys resolved as the reference's main.py resolves them (CPU), and an end-to-end
compress / decompress / verify run (GPU)."""
import numpy as np
import pytest


def _cfg(tmp_path, body):
    p = tmp_path / "exp1.yaml"
    p.write_text(body)
    return p


def test_resolve_config_keys(tmp_path):
    import cli

    p = _cfg(tmp_path, "model:\n  d_model: 256\n  num_layers: 2\n  path: m.bin\ncompression:\n"
                       "  file_to_compress: data/in.bin\n  chunks_count: 7\nexperiments_root: out\nverify: true\n")
    a = cli.parse_args(["--config", str(p), "--no-progress"])
    r = cli.resolve(a, cli.load_config(p))
    assert r["name"] == "exp1"
    assert r["boa_path"] == (tmp_path / "out" / "exp1" / "exp1.boa").resolve()
    assert r["src"] == (tmp_path / "data" / "in.bin").resolve()
    assert r["model_path"] == (tmp_path / "m.bin").resolve()
    assert (r["chunks_count"], r["num_layers"], r["verify"], r["progress"]) == (7, 2, True, False)
    assert r["precision"] == "f32"  # the reference's default "fp32" is plain float32 arithmetic


@pytest.mark.parametrize("flag,mode", [("fp32", "f32"), ("f32", "f32"), ("bf16x3", "bf16x3"), ("bf16w", "bf16w")])
def test_precision_flag_mapping(tmp_path, flag, mode):
    """--precision fp32 (main.py:59, the reference's default) selects the fp32 MFMA mode; the narrower
    split-bfloat16 modes are chosen only by their own names, from the flag or the config key."""
    import cli

    p = _cfg(tmp_path, "file_path: x.bin\n")
    assert cli.resolve(cli.parse_args(["-c", str(p), "--precision", flag]), cli.load_config(p))["precision"] == mode
    q = _cfg(tmp_path, f"file_path: x.bin\nprecision: {flag}\n")
    assert cli.resolve(cli.parse_args(["-c", str(q)]), cli.load_config(q))["precision"] == mode
    with pytest.raises(SystemExit):
        cli.parse_args(["-c", str(p), "--precision", "fp16"])


def test_resolve_defaults_and_rejections(tmp_path):
    import cli

    p = _cfg(tmp_path, "file_path: x.bin\n")
    r = cli.resolve(cli.parse_args(["-c", str(p), "--precision", "bf16w"]), cli.load_config(p))
    assert r["chunks_count"] == 1000 and r["d_model"] == 256 and r["precision"] == "bf16w"
    assert r["boa_path"].name == "exp1.boa" and r["boa_path"].parent.parent.name == "experiments"
    for flag in ("--train-only", "--evaluate", "--comparison-baseline-only"):
        with pytest.raises(SystemExit):
            cli.resolve(cli.parse_args(["-c", str(p), flag]), cli.load_config(p))
    with pytest.raises(SystemExit):
        cli.resolve(cli.parse_args(["-c", str(p), "--device", "cpu"]), cli.load_config(p))


@pytest.mark.gpu
def test_cli_round_trip(gpu, tmp_path, capsys):
    import cli

    data = np.random.default_rng(3).integers(0, 40, 6000).astype(np.uint8).tobytes()
    (tmp_path / "in.bin").write_bytes(data)
    p = _cfg(tmp_path, "model:\n  num_layers: 2\ncompression:\n  file_to_compress: in.bin\n  chunks_count: 5\n")
    assert cli.main(["-c", str(p), "--no-progress", "--verify", "--show-timings"]) == 0
    out = capsys.readouterr().out
    assert "VERIFY: OK" in out and "compression:" in out
    assert (tmp_path / "experiments" / "exp1" / "exp1_decompressed.bin").read_bytes() == data
    assert cli.main(["-c", str(p), "--no-progress", "--decompress-only", "--verify"]) == 0


def test_default_precision_is_fp32():
    """The drop-in model computes in the reference's fp32 arithmetic unless a narrower mode is asked for."""
    import os

    import model

    assert model.DEFAULT_PRECISION == os.environ.get("BOA_PRECISION", "f32")
    assert model.BoaConstrictor(256, 1, 256).precision == model.DEFAULT_PRECISION
