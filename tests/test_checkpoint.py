"""Packed-weights files: save -> load round trips are byte-exact; malformed files raise ValueError.

The reference has no file format (PackedTensor takes in-memory uint8 Tensors, dx12.py:26-30);
the pins here are the round trip itself and the oracle's dequantisation of what comes back.
"""

import json

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x import checkpoint
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor

CASES = [("int4", torch.float16, 128), ("uint4", None, 32), ("fp4_e2m1", torch.float8_e8m0fnu, 32),
         ("fp6_e2m3", torch.float8_e8m0fnu, 32), ("fp6_e3m2", torch.float32, 64), ("fp4_e2m1", torch.float64, 3)]


def make(fmt, sdt, bs, n=7, k=96, seed=0):
    rng = np.random.default_rng(seed)
    bits = FORMATS[fmt][0]
    data = torch.from_numpy(O.pack_codes(rng.integers(0, 1 << bits, (n, k)).astype(np.uint8), bits))
    scales = None
    nb = (k + bs - 1) // bs
    if sdt is torch.float8_e8m0fnu:
        scales = torch.from_numpy(rng.integers(120, 135, (n, nb)).astype(np.uint8)).view(torch.float8_e8m0fnu)
    elif sdt is not None:
        scales = torch.from_numpy(rng.uniform(0.01, 2.0, (n, nb))).to(sdt)
    return PackedTensor(data, fmt, (n, k), scales, bs)


def scales_np(t: PackedTensor):
    if t.scales is None:
        return None
    if t.scales.dtype is torch.float8_e8m0fnu:
        return O.e8m0_decode(t.scales.view(torch.uint8).numpy())
    return t.scales.to(torch.float64).numpy()


def test_round_trip_is_byte_exact(tmp_path):
    tensors = {f"w{i}": make(*case, seed=i) for i, case in enumerate(CASES)}
    tensors["norm"] = torch.randn(96).to(torch.bfloat16)
    tensors["table"] = torch.arange(12, dtype=torch.int32).reshape(3, 4)
    path = tmp_path / "weights.safetensors"
    checkpoint.save(path, tensors, {"model": "test", "layers": 2})
    loaded, meta = checkpoint.load(path)
    assert meta == {"model": "test", "layers": 2}
    assert set(loaded) == set(tensors)
    for name, t in tensors.items():
        got = loaded[name]
        if isinstance(t, PackedTensor):
            assert isinstance(got, PackedTensor)
            assert (got.format, got.shape, got.block_size) == (t.format, t.shape, t.block_size)
            assert torch.equal(got.data, t.data)
            if t.scales is None:
                assert got.scales is None
            else:
                assert got.scales.dtype is t.scales.dtype
                assert torch.equal(got.scales.view(torch.uint8), t.scales.view(torch.uint8))
            # the oracle decodes the loaded file to the same values
            want = O.dequant_f64(t.data.numpy(), t.format, t.shape, scales_np(t), t.block_size)
            have = O.dequant_f64(got.data.numpy(), got.format, got.shape, scales_np(got), got.block_size)
            assert np.array_equal(want, have, equal_nan=True)
        else:
            assert got.dtype is t.dtype and torch.equal(got, t)


def test_malformed_files_raise_value_error(tmp_path):
    from safetensors.torch import save_file

    good = make("fp4_e2m1", torch.float8_e8m0fnu, 32)
    path = tmp_path / "bad.safetensors"
    arrays = {"w": good.data, "w.scales": good.scales}
    cases = [
        ({"tgm.packed": "{not json"}, "corrupt"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp5", "shape": [7, 96], "block_size": 32, "scales": True}})}, "format"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "block_size": 32, "scales": True},
                                    "v": {"format": "int4", "shape": [1, 2], "block_size": 32, "scales": False}})},
         "missing"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [70, 96], "block_size": 32, "scales": True}})},
         "smaller than the declared shape"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "block_size": 16, "scales": True}})},
         "incompatible shape"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "block_size": 32, "scales": True}})}, "shape must be"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96.0], "block_size": 32,
                                          "scales": True}})}, "shape must be"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "scales": True}})},
         "block_size must be"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "block_size": "32",
                                          "scales": True}})}, "block_size must be"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "block_size": 32}})},
         "scales must be"),
        ({"tgm.packed": json.dumps({"w": {"format": "fp4_e2m1", "shape": [7, 96], "block_size": 32,
                                          "scales": False}})}, "declared unscaled"),
        ({"tgm.packed": json.dumps({})}, "no declared packed tensor"),
    ]
    for metadata, message in cases:
        save_file(arrays, str(path), metadata=metadata)
        with pytest.raises(ValueError, match=message):
            checkpoint.load(path)
    with pytest.raises(ValueError, match="may not end"):
        checkpoint.save(path, {"x.scales": torch.zeros(1)})
