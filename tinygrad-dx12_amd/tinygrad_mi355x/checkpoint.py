"""On-disk packed weights: PackedTensor (codes + block scales) in a safetensors file.

The reference takes packed weights only as in-memory uint8 Tensors (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/codegen/decomp/dx12.py:26-30) and has no file format.  Loading a model onto
the packed path needs one, so this module defines it on top of safetensors (a flat header of
named, typed, contiguous arrays that can be memory-mapped and copied to the device in one go):

* a packed tensor ``name`` is stored as two arrays: ``name`` holds the LSB-first bit stream of
  its codes as flat uint8 (the reference's layout, dx12.py:69-77), and ``name.scales`` its
  block scales in their own dtype (E8M0 bytes as ``float8_e8m0fnu``, or f16 / bf16 / f32 / f64);
* the file metadata key ``tgm.packed`` is a JSON object mapping each packed name to
  ``{"format", "shape", "block_size", "scales"}`` (``scales`` false for unscaled tensors);
* every other array is an ordinary dense tensor; the metadata key ``tgm.meta`` carries a
  caller-defined JSON object (a model configuration, for instance).

Round trip: ``load(save(x))`` gives byte-identical codes and scales.  Everything a file
declares is validated on load with the same ValueError checks as PackedTensor itself.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor

PACKED_KEY, META_KEY = "tgm.packed", "tgm.meta"
SCALE_SUFFIX = ".scales"


def save(path: str | Path, tensors: dict[str, PackedTensor | torch.Tensor], meta: dict | None = None) -> None:
    """Write packed and dense tensors (on any device) to ``path``."""
    from safetensors.torch import save_file

    arrays: dict[str, torch.Tensor] = {}
    packed: dict[str, dict] = {}
    for name, t in tensors.items():
        if name.endswith(SCALE_SUFFIX):
            raise ValueError(f"tensor names may not end in {SCALE_SUFFIX!r}: {name!r}")
        if isinstance(t, PackedTensor):
            arrays[name] = t.data.detach().contiguous().cpu()
            if t.scales is not None:
                arrays[name + SCALE_SUFFIX] = t.scales.detach().contiguous().cpu()
            packed[name] = {"format": t.format, "shape": list(t.shape), "block_size": t.block_size,
                            "scales": t.scales is not None}
        elif isinstance(t, torch.Tensor):
            arrays[name] = t.detach().contiguous().cpu()
        else:
            raise ValueError(f"{name!r} is neither a PackedTensor nor a Tensor")
    metadata = {PACKED_KEY: json.dumps(packed, sort_keys=True)}
    if meta is not None:
        metadata[META_KEY] = json.dumps(meta, sort_keys=True)
    save_file(arrays, str(path), metadata=metadata)


def _check_spec(name: str, spec) -> tuple[tuple[int, ...], int, bool]:
    """Validate one ``tgm.packed`` entry's field types; returns (shape, block_size, scaled)."""
    if not isinstance(spec, dict) or spec.get("format") not in FORMATS:
        raise ValueError(f"packed tensor {name!r}: unknown or missing format")
    shape, block, scaled = spec.get("shape"), spec.get("block_size"), spec.get("scales")
    if not isinstance(shape, list) or not all(isinstance(x, int) and not isinstance(x, bool) for x in shape):
        raise ValueError(f"packed tensor {name!r}: shape must be a list of integers, got {shape!r}")
    if not isinstance(block, int) or isinstance(block, bool):
        raise ValueError(f"packed tensor {name!r}: block_size must be an integer, got {block!r}")
    if not isinstance(scaled, bool):
        raise ValueError(f"packed tensor {name!r}: scales must be true or false, got {scaled!r}")
    return tuple(shape), block, scaled


def load(path: str | Path, device: str | torch.device = "cpu") -> tuple[dict[str, PackedTensor | torch.Tensor], dict]:
    """Read a file written by ``save``; returns (tensors, meta) with tensors on ``device``."""
    from safetensors import safe_open

    tensors: dict[str, PackedTensor | torch.Tensor] = {}
    with safe_open(str(path), framework="pt", device=str(device)) as f:
        metadata = f.metadata() or {}
        try:
            packed = json.loads(metadata.get(PACKED_KEY, "{}"))
            meta = json.loads(metadata.get(META_KEY, "{}"))
        except json.JSONDecodeError as error:
            raise ValueError(f"corrupt packed-tensor metadata in {path}: {error}") from error
        if not isinstance(packed, dict) or not isinstance(meta, dict):
            raise ValueError(f"corrupt packed-tensor metadata in {path}")
        names = set(f.keys())
        for name, spec in packed.items():
            shape, block, scaled = _check_spec(name, spec)
            if name not in names or (scaled and name + SCALE_SUFFIX not in names):
                raise ValueError(f"packed tensor {name!r}: missing data or scales array")
            if not scaled and name + SCALE_SUFFIX in names:
                raise ValueError(f"packed tensor {name!r}: declared unscaled but the file holds {name + SCALE_SUFFIX!r}")
            data = f.get_tensor(name)
            scales = f.get_tensor(name + SCALE_SUFFIX) if scaled else None
            tensors[name] = PackedTensor(data, spec["format"], shape, scales, block)
        for name in names:
            if name in tensors or (name.endswith(SCALE_SUFFIX) and name[: -len(SCALE_SUFFIX)] in packed):
                continue
            if name.endswith(SCALE_SUFFIX):
                raise ValueError(f"{name!r} holds block scales of no declared packed tensor")
            tensors[name] = f.get_tensor(name)
    return tensors, meta
