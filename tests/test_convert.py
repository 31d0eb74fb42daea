"""The offline converter's writer contract on small synthetic checkpoints (CPU only): header order
and metadata, quantized tensors equal to the oracle's quantizers bit for bit, untouched tensors
byte-identical, and each refusal of the contract."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from kitchen_amd import convert as C
from oracle import linear, quant


def _source(path, seed=0, extra_meta=None):
    g = torch.Generator().manual_seed(seed)
    tensors = {
        "blocks.0.attn.qkv.weight": (torch.randn(96, 512, generator=g) * 0.02).to(torch.bfloat16),
        "blocks.0.attn.qkv.bias": torch.randn(96, generator=g).to(torch.bfloat16),
        "blocks.0.norm1.weight": torch.ones(512, dtype=torch.bfloat16),
        "blocks.0.mlp.fc1.weight": (torch.randn(128, 256, generator=g) * 0.02).to(torch.float32),
        "blocks.0.mlp.odd.weight": torch.randn(32, 200, generator=g).to(torch.bfloat16),   # K % 256 != 0
        "embed_tokens.weight": torch.randn(50, 256, generator=g).to(torch.bfloat16),
        "conv.weight": torch.randn(8, 4, 3, 3, generator=g).to(torch.float16),
    }
    save_file(tensors, str(path), metadata=extra_meta or {"modelspec.title": "synthetic"})
    return tensors


def _read(path):
    with safe_open(str(path), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def _raw_header(path):
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        return json.loads(f.read(n))


@pytest.mark.parametrize("fmt_name", ["w4a8_asym_g64", "w4a4_sym_g64", "convrot_w4a4", "int8_tensorwise"])
def test_convert_formats(tmp_path, fmt_name):
    src, out = tmp_path / "m.safetensors", tmp_path / "q.safetensors"
    tensors = _source(src)
    fmt = C.make_format(fmt_name)
    manifest = C.convert(src, out, fmt, "cpu")
    got, meta = _read(out)
    assert (tmp_path / "q.quant.json").exists() and not (tmp_path / "q.safetensors.partial").exists()
    quantized = ["blocks.0.attn.qkv.weight", "blocks.0.mlp.fc1.weight"]
    assert manifest["quantized_tensors"] == 2
    qm = json.loads(meta["_quantization_metadata"])
    assert qm["format_version"] == "1.0"
    assert set(qm["layers"]) == {"blocks.0.attn.qkv", "blocks.0.mlp.fc1"}
    assert all(v["format"] == fmt_name for v in qm["layers"].values())
    assert meta["quantization"] == fmt_name and meta["modelspec.title"] == "synthetic"
    # key order: the source's, each quantized weight expanded in place
    keys = [k for k in _raw_header(out) if k != "__metadata__"]
    expect = []
    for k in (k for k in _raw_header(src) if k != "__metadata__"):
        expect += [k] + ([k.removesuffix(".weight") + "." + t for t in
                          {"w4a8_asym_g64": ["weight_scale", "weight_zero"]}.get(fmt_name, ["weight_scale"])]
                         if k in quantized else [])
    assert keys == expect
    # untouched tensors byte-identical
    for k in ("blocks.0.attn.qkv.bias", "blocks.0.norm1.weight", "blocks.0.mlp.odd.weight", "embed_tokens.weight",
              "conv.weight"):
        assert torch.equal(got[k].view(torch.uint8), tensors[k].contiguous().view(torch.uint8)), k
    # quantized tensors: the oracle's quantizers on the same fp32 weight
    for name in quantized:
        w = tensors[name].float().numpy()
        b = name.removesuffix(".weight")
        if fmt_name == "w4a8_asym_g64":
            q, s16, z = quant.quant_weight_u4_asym(linear.rotate_weight(w, 256), 64)
            assert np.array_equal(got[name].numpy(), quant.pack_u4(q))
            assert np.array_equal(got[b + ".weight_scale"].numpy(), s16)
            assert np.array_equal(got[b + ".weight_zero"].numpy(), quant.pack_u4(z))
        elif fmt_name == "w4a4_sym_g64":
            q, s16 = quant.quant_weight_i4_sym_group(linear.rotate_weight(w, 64), 64)
            assert np.array_equal(got[name].numpy(), quant.pack_i4(q))
            assert np.array_equal(got[b + ".weight_scale"].numpy(), s16)
        elif fmt_name == "convrot_w4a4":
            q, s = quant.quant_weight_i4_rowwise(linear.rotate_weight(w, 256))
            assert np.array_equal(got[name].numpy(), quant.pack_i4(q))
            assert np.array_equal(got[b + ".weight_scale"].numpy(), s)
        else:
            q, s = quant.quant_weight_i8_rowwise(linear.rotate_weight(w, 256))
            assert np.array_equal(got[name].numpy(), q)
            assert np.array_equal(got[b + ".weight_scale"].numpy(), s.reshape(-1, 1))


def test_refusals(tmp_path):
    src, out = tmp_path / "m.safetensors", tmp_path / "q.safetensors"
    _source(src)
    fmt = C.make_format("w4a8_asym_g64")
    with pytest.raises(SystemExit, match="output is the source"):
        C.convert(src, src, fmt)
    C.convert(src, out, fmt)
    with pytest.raises(SystemExit, match="exists"):
        C.convert(src, out, fmt)                              # existing output
    out.unlink()
    with pytest.raises(SystemExit, match="exists"):
        C.convert(src, out, fmt)                              # sidecar still there
    (tmp_path / "q.quant.json").unlink()
    (tmp_path / "q.safetensors.partial").write_bytes(b"x")
    with pytest.raises(SystemExit, match="stale"):
        C.convert(src, out, fmt)
    (tmp_path / "q.safetensors.partial").unlink()
    # an already quantized source, both markers
    qsrc = tmp_path / "qq.safetensors"
    _source(qsrc, extra_meta={"_quantization_metadata": "{}"})
    with pytest.raises(SystemExit, match="already"):
        C.convert(qsrc, tmp_path / "o1.safetensors", fmt)
    msrc = tmp_path / "mk.safetensors"
    save_file({"a.weight": torch.zeros(4, 256), "a.comfy_quant": torch.zeros(1, dtype=torch.uint8)}, str(msrc))
    with pytest.raises(SystemExit, match="comfy_quant"):
        C.convert(msrc, tmp_path / "o2.safetensors", fmt)
    # nothing compatible
    nsrc = tmp_path / "n.safetensors"
    save_file({"a.weight": torch.zeros(4, 100)}, str(nsrc))
    with pytest.raises(SystemExit, match="no layer"):
        C.convert(nsrc, tmp_path / "o3.safetensors", fmt)
    assert not list(tmp_path.glob("*.partial"))


def test_failure_midway_leaves_nothing(tmp_path, monkeypatch):
    src, out = tmp_path / "m.safetensors", tmp_path / "q.safetensors"
    _source(src)
    fmt = C.make_format("convrot_w4a4")
    calls = {"n": 0}
    real = C.Format.quantize

    def failing(self, w):
        calls["n"] += 1
        if calls["n"] == 2:
            raise RuntimeError("device lost")
        return real(self, w)

    monkeypatch.setattr(C.Format, "quantize", failing)
    with pytest.raises(RuntimeError):
        C.convert(src, out, fmt)
    assert not out.exists() and not (tmp_path / "q.quant.json").exists()
    assert not list(tmp_path.glob("*.partial"))


def test_cli_dry_run_and_write(tmp_path, capsys):
    src = tmp_path / "m.safetensors"
    _source(src)
    assert C.main([str(src), "--format", "int8_tensorwise", "--device", "cpu", "--dry-run"]) == 0
    assert "2 of 7 tensors" in capsys.readouterr().out
    assert C.main([str(src), "--format", "int8_tensorwise", "--device", "cpu", "--include", "mlp"]) == 0
    got, meta = _read(tmp_path / "m_int8_tensorwise.safetensors")
    assert set(json.loads(meta["_quantization_metadata"])["layers"]) == {"blocks.0.mlp.fc1"}
