"""Strict loading of calibrated K/V rotation artefacts (reference rotations.py:1-53).

Checkpoint formats accepted (as the reference): a [layers, D, D] tensor, or a dict
``{"layers": {index: matrix | {"rotation": matrix}}}`` / ``{index: ...}``. Files are read with
``torch.load(weights_only=True)`` only. ``get_rotation`` validates shape, finiteness and
orthogonality on the checkpoint's fp32 values before the bf16 device copy.
"""

from __future__ import annotations

import re
from functools import lru_cache

import torch


def layer_index(name):
    """Global decoder layer index of a module name (``...layers.<i>...``)."""
    match = re.search(r"(?:^|\.)layers\.(\d+)(?:\.|$)", name)
    if match is None:
        raise ValueError(f"Cannot resolve global decoder layer index: {name}")
    return int(match.group(1))


def _table(source, path):
    if torch.is_tensor(source) and source.ndim == 3:
        items = enumerate(source)
    elif isinstance(source, dict):
        items = source.get("layers", source).items()
    else:
        raise ValueError(f"Unsupported rotation checkpoint format: {path}")
    result = {}
    for key, entry in items:
        matrix = entry["rotation"] if isinstance(entry, dict) else entry
        if not torch.is_tensor(matrix):
            raise ValueError(f"Invalid matrix for layer {key} in {path}")
        result[int(key)] = matrix.float().contiguous()
    return result


@lru_cache(maxsize=4)
def load_checkpoint(path):
    if not path:
        raise ValueError("Calibrated D256 K/V rotation paths are required")
    return _table(torch.load(path, map_location="cpu", weights_only=True), path)


def get_rotation(path, name, device, dim=256):
    """The layer's rotation as contiguous bf16 on ``device`` (reference rotations.py:36-53)."""
    index = layer_index(name)
    table = load_checkpoint(path)
    if index not in table:
        raise ValueError(f"Missing rotation for {name} (layer {index}) in {path}")
    matrix = table[index]
    if tuple(matrix.shape) != (dim, dim):
        raise ValueError(f"Expected D{dim} rotation for {name}; got {tuple(matrix.shape)}")
    if not torch.isfinite(matrix).all():
        raise ValueError(f"Nonfinite rotation for {name}")
    identity = torch.eye(dim, dtype=matrix.dtype)
    if not torch.allclose(matrix.T @ matrix, identity, atol=0.015, rtol=0.015):
        raise ValueError(f"Rotation for {name} is not orthogonal")
    return matrix.to(device=device, dtype=torch.bfloat16).contiguous()


def save_rotations(path, rotations):
    """Write ``{layer index: [D, D] matrix}`` in the format ``load_checkpoint`` reads."""
    torch.save({"layers": {int(k): {"rotation": v.detach().float().cpu().contiguous()}
                           for k, v in rotations.items()}}, path)
