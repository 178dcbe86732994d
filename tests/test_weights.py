"""Safetensors reader and backbone weight loader (models/weights.rs:26-104,
196-215): header validation on the CPU, device conversion and the golden
fixture loaded from disk on the GPU."""
import json
import struct

import numpy as np
import pytest
import torch

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def clef():
    import clef_hip
    clef_hip.lib()
    return clef_hip


def _raw(path, header, data=b"", length=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h) if length is None else length) + h + data)
    return path


def test_reader_lists_tensors_of_a_valid_file(clef, tmp_path):
    from safetensors.torch import save_file
    p = tmp_path / "ok.safetensors"
    save_file({"a": torch.zeros(3, 4, dtype=torch.bfloat16), "b": torch.ones(5, dtype=torch.float16),
               "c": torch.arange(6, dtype=torch.float32).reshape(2, 3)}, str(p), metadata={"format": "pt"})
    with clef.SafeTensors(p) as st:
        assert st.tensors() == {"a": ("BF16", (3, 4)), "b": ("F16", (5,)), "c": ("F32", (2, 3))}


@pytest.mark.parametrize("case", ["short", "huge_header", "truncated", "not_object", "duplicate", "dtype",
                                  "beyond", "bytes", "gap", "overlap", "trailing", "entries"])
def test_reader_rejects_malformed_headers(clef, tmp_path, case):
    """weights.rs:196-215 limits and the safetensors layout rules."""
    p = tmp_path / f"{case}.safetensors"
    t = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    if case == "short":
        p.write_bytes(b"\x00\x00\x00")
    elif case == "huge_header":
        _raw(p, b"{}", length=1024 * 1024 + 1)
    elif case == "truncated":
        _raw(p, b'{"x": {}}', length=64)
    elif case == "not_object":
        _raw(p, b"[1, 2]")
    elif case == "duplicate":
        _raw(p, b'{"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},'
                b' "x": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}', b"\x00" * 8)
    elif case == "dtype":
        _raw(p, {"x": {"dtype": "I64", "shape": [1], "data_offsets": [0, 8]}}, b"\x00" * 8)
    elif case == "beyond":
        _raw(p, {"x": t}, b"\x00" * 4)
    elif case == "bytes":
        _raw(p, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\x00" * 8)
    elif case == "gap":
        _raw(p, {"x": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\x00" * 8)
    elif case == "overlap":
        _raw(p, {"x": t, "y": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}, b"\x00" * 12)
    elif case == "trailing":
        _raw(p, json.dumps({"x": t}).encode() + b" junk", b"\x00" * 8)
    elif case == "entries":
        hdr = {f"t{i}": {"dtype": "F32", "shape": [1], "data_offsets": [4 * i, 4 * i + 4]} for i in range(2049)}
        _raw(p, hdr, b"\x00" * (4 * 2049))
    with pytest.raises(clef.ClefError):
        clef.SafeTensors(p)


def test_loader_rejects_unconsumed_and_misshapen_tensors(clef, tmp_path, golden_dir):
    """Checks made before any tensor is loaded (weights.rs:52-63, 184-189)."""
    from safetensors.torch import save_file
    cfg = json.loads((golden_dir / "backbone-config.json").read_text())
    p = tmp_path / "extra.safetensors"
    save_file({"model.language_model.layers.0.unexpected": torch.zeros(2)}, str(p))
    with pytest.raises(clef.ClefError, match="unconsumed"):
        clef.load_backbone_weights(cfg, p)
    save_file({"model.language_model.norm.weight": torch.zeros(cfg["hidden_size"] + 1)}, str(p))
    with pytest.raises(clef.ClefError, match="shape"):
        clef.load_backbone_weights(cfg, p)


@gpu
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dst", [torch.float16, torch.float32])
def test_device_conversion_rounds_as_torch(clef, tmp_path, src, dst):
    """BF16 -> F32 and F16 -> F32 exact; -> F16 round to nearest even (torch's
    casts from the exact f32 value), including subnormal and overflowing values."""
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4097, generator=g) * torch.logspace(-9, 6, 4097)
    x[:4] = torch.tensor([0.0, -0.0, 70000.0, 6.1e-5])
    x = x.to(src)
    p = tmp_path / "conv.safetensors"
    save_file({"x": x}, str(p))
    with clef.SafeTensors(p) as st:
        got = st.load("x", dst)
    assert torch.equal(got.cpu(), x.float().to(dst))


@gpu
@pytest.mark.parametrize("profile", ["f32", "mixed"])
def test_golden_fixture_loaded_from_disk(clef, golden_dir, profile):
    """The reference's synthetic checkpoint through the loader reproduces its
    golden hidden states (mod.rs:75-111 tolerance for f32)."""
    from safetensors.numpy import load_file
    cfg = json.loads((golden_dir / "backbone-config.json").read_text())
    exp = load_file(str(golden_dir / "backbone-output.safetensors"))["hidden"].astype(np.float64)
    b = clef.Backbone.from_safetensors(cfg, golden_dir / "backbone.safetensors", profile=profile)
    got = b.prefill(np.arange(20))[0].cpu().numpy().astype(np.float64)
    if profile == "f32":
        tol = 1e-5 + 1e-4 * np.abs(exp)
    else:
        tol = 2e-2 * np.abs(exp).max() + 2e-2 * np.abs(exp)
    assert (np.abs(got - exp) <= tol).all()


@gpu
def test_loader_reports_a_missing_tensor(clef, tmp_path, golden_dir):
    from safetensors.torch import load_file, save_file
    cfg = json.loads((golden_dir / "backbone-config.json").read_text())
    w = load_file(str(golden_dir / "backbone.safetensors"))
    w.pop("model.language_model.layers.3.self_attn.k_norm.weight")
    p = tmp_path / "missing.safetensors"
    save_file(w, str(p))
    with pytest.raises(clef.ClefError, match="missing"):
        clef.load_backbone_weights(cfg, p)
