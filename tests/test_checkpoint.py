"""MLX-affine safetensors checkpoints read without repacking: round trip,
per-layer quantization overrides, and named refusals. CPU only."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

from kernelverify_amd.checkpoint import (
    CheckpointError,
    layer_quantization,
    load_quantized_linears,
    quantized_layers,
    save_quantized_linears,
)
from oracle.quant_contract import QuantContract, canonical_quantize, dequantize, pack_codes


def _art(d_out, d_in, bits, seed):
    w = (np.random.default_rng(seed).standard_normal((d_out, d_in)) * 0.02).astype(np.float16)
    art = canonical_quantize(w, QuantContract(bits=bits, group_size=64))
    return art, (pack_codes(art.q, bits), art.scales, art.biases)


def test_round_trip_is_byte_identical_and_computes_the_product(tmp_path):
    a, ta = _art(96, 256, 4, 1)
    b, tb = _art(64, 128, 4, 2)
    save_quantized_linears(tmp_path / "model.safetensors",
                           {"layers.0.mlp.up_proj": ta, "layers.0.mlp.down_proj": tb}, bits=4)
    layers = load_quantized_linears(tmp_path, device="cpu")
    assert sorted(layers) == ["layers.0.mlp.down_proj", "layers.0.mlp.up_proj"]
    up = layers["layers.0.mlp.up_proj"]
    assert np.array_equal(up.weight.numpy().view(np.uint32), ta[0])
    assert np.array_equal(up.scales.numpy(), ta[1]) and np.array_equal(up.biases.numpy(), ta[2])
    assert (up.bits, up.d_out, up.d_in) == (4, 96, 256)
    x = np.random.default_rng(3).standard_normal((2, 256)).astype(np.float32)
    ref = x.astype(np.float64) @ dequantize(a).astype(np.float64).T
    got = up(torch.from_numpy(x)).numpy()
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_per_layer_overrides_and_unquantized_layers(tmp_path):
    _, t4 = _art(64, 128, 4, 1)
    _, t8 = _art(64, 128, 8, 2)
    tensors = {"q.weight": t4[0], "q.scales": t4[1], "q.biases": t4[2],
               "o.weight": t8[0], "o.scales": t8[1], "o.biases": t8[2],
               "norm.weight": np.ones(64, np.float16),
               "skip.weight": t4[0], "skip.scales": t4[1], "skip.biases": t4[2]}
    save_file(tensors, str(tmp_path / "m.safetensors"))
    block = {"group_size": 64, "bits": 4, "o": {"bits": 8}, "skip": False}
    (tmp_path / "config.json").write_text(json.dumps({"quantization": block}))
    assert quantized_layers(tensors) == ["o", "q", "skip"]
    assert layer_quantization(block, "o") == (8, 64) and layer_quantization(block, "skip") is None
    layers = load_quantized_linears(tmp_path, device="cpu")
    assert sorted(layers) == ["o", "q"] and layers["o"].bits == 8 and layers["q"].bits == 4


def test_refusals_name_the_layer(tmp_path):
    _, t4 = _art(64, 128, 4, 1)
    save_file({"x.weight": t4[0].astype(np.int64), "x.scales": t4[1], "x.biases": t4[2]},
              str(tmp_path / "a.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4}}))
    with pytest.raises(CheckpointError, match="x.weight must be uint32"):
        load_quantized_linears(tmp_path, device="cpu")
    (tmp_path / "a.safetensors").unlink()
    save_file({"x.weight": t4[0], "x.scales": t4[1], "x.biases": t4[2]},
              str(tmp_path / "a.safetensors"))
    with pytest.raises(CheckpointError, match="8-bit d_in=128"):
        load_quantized_linears(tmp_path, config={"quantization": {"bits": 8}}, device="cpu")
    with pytest.raises(CheckpointError, match="no quantization block"):
        load_quantized_linears(tmp_path, config={"model_type": "llama"}, device="cpu")
