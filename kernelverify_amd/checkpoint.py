"""MLX-affine quantized checkpoints on disk, read without repacking
(reference: kernelverify/pack/wide_qmv.py:41-46, the artefact layout the
pack kernels read; mlx-lm's safetensors checkpoints of quantized models).

A quantized linear `<name>` is stored as three tensors:

    <name>.weight   uint32 (d_out, d_in * bits / 32)   little-endian code
                    stream, lowest code in the lowest bits, codes may straddle
                    words below 4 bits
    <name>.scales   fp16   (d_out, d_in / group_size)
    <name>.biases   fp16   (d_out, d_in / group_size)

plus an optional fp16 `<name>.bias`. The checkpoint's `config.json` carries
`"quantization": {"group_size": 64, "bits": 4, ...}`, where a key naming a
layer overrides bits or group size for that layer (or is `false` for a layer
left unquantized). These bytes are the kernels' own layout, so loading is a
copy to the device and nothing is repacked.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

SUFFIXES = ("weight", "scales", "biases")


class CheckpointError(ValueError):
    """A tensor set that is not an MLX-affine quantized linear, with the name."""


def quantization_config(config) -> dict:
    """The `quantization` block of a config dict or `config.json` path."""
    if isinstance(config, (str, Path)):
        config = json.loads(Path(config).read_text())
    block = config.get("quantization", config.get("quantization_config"))
    if not isinstance(block, dict) or "bits" not in block:
        raise CheckpointError("config has no quantization block with 'bits'")
    return block


def layer_quantization(block: dict, name: str) -> tuple[int, int] | None:
    """(bits, group_size) of layer `name`, or None where the config leaves
    it unquantized; a per-layer entry overrides the defaults."""
    own = block.get(name)
    if own is False:
        return None
    bits, group = int(block["bits"]), int(block.get("group_size", 64))
    if isinstance(own, dict):
        bits, group = int(own.get("bits", bits)), int(own.get("group_size", group))
    return bits, group


def quantized_layers(tensors: dict) -> list[str]:
    """Names that have a full weight / scales / biases triple."""
    names = {k.rsplit(".", 1)[0] for k in tensors if k.endswith(".scales")}
    return sorted(n for n in names if all(f"{n}.{s}" in tensors for s in SUFFIXES))


def check_layer(name: str, tensors: dict, bits: int, group_size: int) -> tuple[int, int]:
    """(d_out, d_in) after checking dtypes and shapes against the layout."""
    w, s, b = (tensors[f"{name}.{k}"] for k in SUFFIXES)
    if w.dtype != np.uint32 or w.ndim != 2:
        raise CheckpointError(f"{name}.weight must be uint32 (d_out, words), got {w.dtype} "
                              f"{w.shape}")
    for label, t in (("scales", s), ("biases", b)):
        if t.dtype != np.float16 or t.ndim != 2:
            raise CheckpointError(f"{name}.{label} must be fp16 (d_out, groups), got {t.dtype}")
    d_out, d_in = s.shape[0], s.shape[1] * group_size  # rows are the output dimension
    if b.shape != s.shape or w.shape[0] != d_out:
        raise CheckpointError(f"{name}: weight {w.shape}, scales {s.shape}, biases {b.shape} "
                              "disagree on d_out")
    if w.shape[1] * 32 != d_in * bits:
        raise CheckpointError(f"{name}: {w.shape[1]} words per row, {bits}-bit d_in={d_in} "
                              f"(group {group_size}) needs {d_in * bits / 32:g}")
    return d_out, d_in


def read_tensors(path) -> dict:
    """Every tensor of one or more .safetensors files as numpy arrays (no
    code runs from the file)."""
    from safetensors.numpy import load_file

    paths = [Path(path)] if Path(path).is_file() else sorted(Path(path).glob("*.safetensors"))
    if not paths:
        raise CheckpointError(f"no .safetensors under {path}")
    tensors: dict = {}
    for p in paths:
        tensors.update(load_file(str(p)))
    return tensors


def load_quantized_linears(path, config=None, device="cuda") -> dict:
    """{name: serving.QuantizedLinear} for every quantized linear of a
    checkpoint file or directory; `config` defaults to the directory's
    config.json. Tensors move to `device` as they are."""
    import torch

    from kernelverify_amd.serving import QuantizedLinear

    root = Path(path) if Path(path).is_dir() else Path(path).parent
    block = quantization_config(config if config is not None else root / "config.json")
    tensors = read_tensors(path)
    layers = {}
    for name in quantized_layers(tensors):
        q = layer_quantization(block, name)
        if q is None:
            continue
        bits, group = q
        check_layer(name, tensors, bits, group)
        as_t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
        bias = tensors.get(f"{name}.bias")
        layers[name] = QuantizedLinear(
            as_t(tensors[f"{name}.weight"].view(np.int32)), as_t(tensors[f"{name}.scales"]),
            as_t(tensors[f"{name}.biases"]), bits,
            bias=None if bias is None else as_t(bias), group_size=group)
    return layers


def save_quantized_linears(path, layers: dict, bits: int, group_size: int = 64) -> None:
    """Write `layers` ({name: (w_q uint32, scales fp16, biases fp16)}) in the
    same layout, and a config.json beside it."""
    from safetensors.numpy import save_file

    tensors = {}
    for name, (w, s, b) in layers.items():
        tensors[f"{name}.weight"] = np.ascontiguousarray(w, dtype=np.uint32)
        tensors[f"{name}.scales"] = np.ascontiguousarray(s, dtype=np.float16)
        tensors[f"{name}.biases"] = np.ascontiguousarray(b, dtype=np.float16)
        check_layer(name, tensors, bits, group_size)
    path = Path(path)
    save_file(tensors, str(path))
    (path.parent / "config.json").write_text(json.dumps(
        {"quantization": {"group_size": group_size, "bits": bits}}, indent=1) + "\n")
