"""Offline converter: a high-precision .safetensors checkpoint -> a quantized one this path runs.

    python -m kitchen_amd.convert SRC.safetensors --format w4a8_asym_g64 [--output OUT]
           [--convrot-groupsize 256] [--group-size 64] [--device cuda|cpu]
           [--include REGEX] [--exclude REGEX] [--dry-run]

The converters of the reference (`tools/quant_w4a8.py:91-168`, `tools/quant_w4a4.py:129-223`)
select the Linear weights, quantize each one on the device and stream the result into a new file.
Their shared writer contract (`tools/_conversion.py:1-60`) is kept here part for part:

    1. refuse source == output, an existing output and an existing sidecar
    2. refuse an already quantized source (`_quantization_metadata` in `__metadata__`, or
       per-layer `.comfy_quant` tensors, `_conversion.py:245-262`)
    3. refuse a stale `.partial`
    4. plan the whole header, every `data_offsets`, before writing a byte: the output shapes are
       analytic (`_formats.py` `tensors()`), so nothing has to be quantized to know them
    5. stream: untouched tensors are copied byte for byte, quantized layers are produced one at a
       time (peak memory ~3 x the largest tensor)
    6. check bytes written == bytes planned
    7. flush + fsync + os.replace, sidecar first, `.partial` removed on any failure
    8. check free disk space first

Output `__metadata__`: the source's, then `_quantization_metadata` = JSON
{"format_version": "1.0", "layers": {layer: config}} and `quantization` = the format name, in that
key order (`_formats.py:279-293`). Formats (tensor names per layer `<l>`):

    convrot_w4a4      <l>.weight I8 [N, K/2], <l>.weight_scale F32 [N]        (_formats.py:53-76)
    int8_tensorwise   <l>.weight I8 [N, K],   <l>.weight_scale F32 [N, 1]     (_formats.py:128-167)
    w4a8_asym_g64     <l>.weight U8 [N, K/2] uint4 codes, <l>.weight_scale F16 [N, K/G],
                      <l>.weight_zero U8 [N, ceil(K/G/2)] packed uint4 zero-points  (configs' W4A8)
    w4a4_sym_g64      <l>.weight I8 [N, K/2], <l>.weight_scale F16 [N, K/G]   (configs' W4A4)

The weight math is kitchen_amd.weights (the HIP quantizer for --device cuda, torch fp32 on the
CPU otherwise; bit-identical codes either way). comfy-kitchen's codebook `asym_w4a8_int8` fitter is not reproduced (it is not in
the reference tree); files in that format are read by w4a8_int8_linear, not written here.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import shutil
import struct
import sys
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import torch

from . import weights as W

FORMAT_VERSION = "1.0"
GIB = 1024 ** 3
CHUNK = 16 * 1024 ** 2

DTYPE_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "I16": 2, "F16": 2, "BF16": 2,
               "I32": 4, "F32": 4, "I64": 8, "F64": 8}
TORCH_DTYPES = {"U8": torch.uint8, "I8": torch.int8, "I16": torch.int16, "I32": torch.int32, "I64": torch.int64,
                "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32, "F64": torch.float64,
                "BOOL": torch.bool}
HEADER_DTYPE = {torch.uint8: "U8", torch.int8: "I8", torch.int16: "I16", torch.int32: "I32", torch.float16: "F16",
                torch.bfloat16: "BF16", torch.float32: "F32"}
SOURCE_DTYPES = frozenset({"BF16", "F16", "F32"})
DEFAULT_EXCLUDE = r"(?i)(embed|norm)"


def _base(name: str) -> str:
    return name.removesuffix(".weight")


def _nbytes(dtype: str, shape) -> int:
    return math.prod(int(d) for d in shape) * DTYPE_BYTES[dtype]


# --------------------------------------------------------------------------- formats

@dataclass(frozen=True)
class Format:
    name: str
    convrot_groupsize: int | None
    group_size: int | None = None

    def accepts(self, shape) -> bool:
        if len(shape) != 2:
            return False
        k = shape[1]
        if k % 2 or (self.convrot_groupsize and k % self.convrot_groupsize):
            return False
        return not self.group_size or k % self.group_size == 0

    def tensors(self, name: str, shape) -> list[tuple[str, str, list[int]]]:
        n, k = (int(d) for d in shape)
        b = _base(name)
        if self.name == "convrot_w4a4":
            return [(name, "I8", [n, k // 2]), (f"{b}.weight_scale", "F32", [n])]
        if self.name == "int8_tensorwise":
            return [(name, "I8", [n, k]), (f"{b}.weight_scale", "F32", [n, 1])]
        g = k // self.group_size
        if self.name == "w4a8_asym_g64":
            return [(name, "U8", [n, k // 2]), (f"{b}.weight_scale", "F16", [n, g]),
                    (f"{b}.weight_zero", "U8", [n, (g + 1) // 2])]
        if self.name == "w4a4_sym_g64":
            return [(name, "I8", [n, k // 2]), (f"{b}.weight_scale", "F16", [n, g])]
        raise ValueError(f"unknown format {self.name!r}")

    def layer_config(self) -> dict:
        cfg = {"format": self.name}
        if self.name == "int8_tensorwise":
            cfg["convrot"] = bool(self.convrot_groupsize)
        if self.group_size:
            cfg["group_size"] = self.group_size
        cfg["convrot_groupsize"] = self.convrot_groupsize or 0
        return cfg

    def quantize(self, weight: torch.Tensor) -> list[torch.Tensor]:
        cg = self.convrot_groupsize
        if self.name == "convrot_w4a4":
            return list(W.quantize_convrot_w4a4_weight(weight, cg, 64))
        if self.name == "int8_tensorwise":
            return list(W.quantize_int8_convrot_weight(weight, cg))
        if self.name == "w4a8_asym_g64":
            return list(W.quantize_w4a8_asym_weight(weight, self.group_size, cg))
        if self.name == "w4a4_sym_g64":
            return list(W.quantize_w4a4_group_weight(weight, self.group_size, cg))
        raise ValueError(f"unknown format {self.name!r}")


def make_format(name: str, convrot_groupsize: int | None = None, group_size: int | None = None) -> Format:
    defaults = {"convrot_w4a4": (256, None), "int8_tensorwise": (256, None), "w4a8_asym_g64": (256, 64),
                "w4a4_sym_g64": (64, 64)}
    if name not in defaults:
        raise ValueError(f"format must be one of {sorted(defaults)}, got {name!r}")
    cg, gs = defaults[name]
    cg = cg if convrot_groupsize is None else (convrot_groupsize or None)
    gs = gs if group_size is None or gs is None else group_size
    if name in ("w4a8_asym_g64", "w4a4_sym_g64") and gs != 64:
        raise ValueError("the group GEMM takes group_size 64")
    if name != "int8_tensorwise" and not cg:
        raise ValueError(f"{name} needs a convrot group size")
    return Format(name, cg, gs)


# --------------------------------------------------------------------------- safetensors I/O

def read_header(path: Path) -> tuple[dict, dict, int]:
    """(tensor entries in file order, __metadata__, byte offset of the data section)."""
    with open(path, "rb") as f:
        (size,) = struct.unpack("<Q", f.read(8))
        raw = json.loads(f.read(size))
    meta = raw.pop("__metadata__", {}) or {}
    return raw, meta, 8 + size


def read_tensor(path: Path, info: dict, data_start: int) -> torch.Tensor:
    begin, end = info["data_offsets"]
    with open(path, "rb") as f:
        f.seek(data_start + begin)
        buf = bytearray(f.read(end - begin))
    t = torch.frombuffer(buf, dtype=TORCH_DTYPES[info["dtype"]]) if buf else torch.empty(0, dtype=TORCH_DTYPES[info["dtype"]])
    return t.reshape(info["shape"])


@dataclass
class Entry:
    key: str
    dtype: str
    shape: list[int]
    nbytes: int
    copy_from: int | None = None        # source byte offset (verbatim copy)
    layer: str | None = None            # weight name whose quantization produces this tensor
    index: int = 0                      # position in that layer's output list


def plan(header: dict, formats: dict[str, Format]) -> list[Entry]:
    entries = []
    for name, info in header.items():
        fmt = formats.get(name)
        if fmt is None:
            begin, end = info["data_offsets"]
            entries.append(Entry(name, info["dtype"], list(info["shape"]), end - begin, copy_from=begin))
        else:
            for i, (key, dt, shape) in enumerate(fmt.tensors(name, info["shape"])):
                entries.append(Entry(key, dt, shape, _nbytes(dt, shape), layer=name, index=i))
    return entries


def build_header(entries: list[Entry], metadata: dict) -> bytes:
    hdr, off = {}, 0
    for e in entries:
        hdr[e.key] = {"dtype": e.dtype, "shape": e.shape, "data_offsets": [off, off + e.nbytes]}
        off += e.nbytes
    hdr["__metadata__"] = {k: str(v) for k, v in metadata.items()}
    text = json.dumps(hdr, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)                     # data section starts 8-byte aligned
    return struct.pack("<Q", len(text)) + text


def quant_metadata(metadata: dict, formats: dict[str, Format], quantization: str) -> dict:
    out = dict(metadata)
    layers = {_base(name): fmt.layer_config() for name, fmt in formats.items()}
    out["_quantization_metadata"] = json.dumps({"format_version": FORMAT_VERSION, "layers": layers},
                                               separators=(",", ":"))
    out["quantization"] = quantization
    return out


# --------------------------------------------------------------------------- the conversion

class ConversionError(SystemExit):
    pass


def select_layers(header: dict, fmt: Format, include: str | None, exclude: str | None) -> list[str]:
    inc = re.compile(include) if include else None
    exc = re.compile(exclude) if exclude else None
    out = []
    for name, info in header.items():
        if not name.endswith(".weight") or info["dtype"] not in SOURCE_DTYPES or not fmt.accepts(info["shape"]):
            continue
        if inc is not None and not inc.search(name):
            continue
        if exc is not None and exc.search(name):
            continue
        out.append(name)
    return out


def refuse_unsafe(source: Path, output: Path, sidecar: Path, header: dict, metadata: dict) -> None:
    if source.resolve() == output.resolve():
        raise ConversionError("refusing: output is the source")
    for p in (output, sidecar):
        if p.exists():
            raise ConversionError(f"refusing: {p} exists")
    partial = output.with_name(output.name + ".partial")
    if partial.exists():
        raise ConversionError(f"refusing: stale {partial} from an interrupted run; remove it first")
    if metadata.get("_quantization_metadata"):
        raise ConversionError("refusing: the source already carries _quantization_metadata")
    if any(name.endswith(".comfy_quant") for name in header):
        raise ConversionError("refusing: the source holds per-layer '.comfy_quant' markers, so it is already quantized")


def convert(source: Path, output: Path, fmt: Format, device: str = "cpu", include: str | None = None,
            exclude: str | None = DEFAULT_EXCLUDE, progress: Callable[[int, int, str], None] | None = None) -> dict:
    """Run the whole contract; returns the sidecar manifest."""
    started = time.perf_counter()
    source, output = Path(source), Path(output)
    sidecar = output.with_suffix(".quant.json")
    header, metadata, data_start = read_header(source)
    refuse_unsafe(source, output, sidecar, header, metadata)
    selected = select_layers(header, fmt, include, exclude)
    if not selected:
        raise ConversionError(f"no layer of {source} is compatible with {fmt.name}")
    formats = {name: fmt for name in selected}
    entries = plan(header, formats)
    head = build_header(entries, quant_metadata(metadata, formats, fmt.name))
    planned = len(head) + sum(e.nbytes for e in entries)
    free = shutil.disk_usage(output.parent).free
    if free < planned + GIB // 64:
        raise ConversionError(f"refusing: {planned} bytes planned, {free} free on {output.parent}")

    partial = output.with_name(output.name + ".partial")
    side_partial = sidecar.with_name(sidecar.name + ".partial")
    written = 0
    try:
        with open(partial, "xb") as out, open(source, "rb") as src:
            out.write(head)
            written += len(head)
            held: list[torch.Tensor] = []
            for i, e in enumerate(entries):
                if e.copy_from is not None:
                    src.seek(data_start + e.copy_from)
                    left = e.nbytes
                    while left:
                        chunk = src.read(min(CHUNK, left))
                        if not chunk:
                            raise ConversionError(f"{source} ends inside {e.key}")
                        out.write(chunk)
                        left -= len(chunk)
                    written += e.nbytes
                    continue
                if e.index == 0:
                    w = read_tensor(source, header[e.layer], data_start).to(device=device, dtype=torch.float32)
                    held = [t.detach().to("cpu").contiguous() for t in fmt.quantize(w)]
                    del w
                    if progress:
                        progress(selected.index(e.layer) + 1, len(selected), e.layer)
                t = held[e.index]
                if HEADER_DTYPE.get(t.dtype) != e.dtype or list(t.shape) != e.shape:
                    raise ConversionError(f"{e.key}: produced {t.dtype} {list(t.shape)}, planned {e.dtype} {e.shape}")
                data = t.view(torch.uint8).numpy().tobytes() if t.numel() else b""
                if len(data) != e.nbytes:
                    raise ConversionError(f"{e.key}: {len(data)} bytes produced, {e.nbytes} planned")
                out.write(data)
                written += len(data)
            if written != planned:
                raise ConversionError(f"wrote {written} bytes, planned {planned}")
            out.flush()
            os.fsync(out.fileno())
        manifest = {
            "source": str(source), "source_size": source.stat().st_size, "output": str(output),
            "output_size": planned, "quantization": fmt.name, "layer_config": fmt.layer_config(),
            "quantized_tensors": len(selected), "preserved_tensors": len(header) - len(selected),
            "device": str(device), "torch_version": torch.__version__,
            "conversion_seconds": round(time.perf_counter() - started, 3),
        }
        with open(side_partial, "x") as f:
            json.dump(manifest, f, indent=1)
            f.flush()
            os.fsync(f.fileno())
        os.replace(side_partial, sidecar)
        try:
            os.replace(partial, output)
        except BaseException:
            sidecar.unlink(missing_ok=True)
            raise
        return manifest
    finally:
        partial.unlink(missing_ok=True)
        side_partial.unlink(missing_ok=True)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("input", type=Path)
    ap.add_argument("--format", required=True, choices=["w4a8_asym_g64", "w4a4_sym_g64", "convrot_w4a4",
                                                        "int8_tensorwise"])
    ap.add_argument("--output", type=Path)
    ap.add_argument("--convrot-groupsize", type=int, default=None, help="Hadamard block (0 = none, int8 only)")
    ap.add_argument("--group-size", type=int, default=None)
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--include", default=None, help="only weights whose name matches this regex")
    ap.add_argument("--exclude", default=DEFAULT_EXCLUDE, help="skip weights whose name matches this regex")
    ap.add_argument("--dry-run", action="store_true")
    args = ap.parse_args(argv)
    src = args.input
    if not src.is_file() or src.suffix.lower() != ".safetensors":
        raise ConversionError("input must be an existing .safetensors file")
    fmt = make_format(args.format, args.convrot_groupsize, args.group_size)
    out = args.output or src.with_name(f"{src.stem}_{fmt.name}.safetensors")
    if args.dry_run:
        header, _, _ = read_header(src)
        sel = select_layers(header, fmt, args.include, args.exclude)
        print(f"{len(sel)} of {len(header)} tensors would be quantized to {fmt.name} -> {out}")
        for name in sel[:10]:
            print(f"  {name}: {header[name]['shape']} {header[name]['dtype']}")
        return 0

    def progress(i, n, name):
        if i % 48 == 0 or i == n:
            print(f"[{i}/{n}] quantized {name}", flush=True)

    m = convert(src, out, fmt, args.device, args.include, args.exclude, progress)
    print(f"wrote {out} ({m['output_size']} bytes, {m['quantized_tensors']} layers) in {m['conversion_seconds']} s")
    return 0


if __name__ == "__main__":
    sys.exit(main())
