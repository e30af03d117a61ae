"""Calibrated K/V rotation artefacts: load once, validate, hand each layer its matrix.

Behaviour follows oscar_ascend/rotations.py:1-53 (reference); the code is this package's own.
An artefact is a ``torch.save`` file read with ``weights_only=True`` (nothing in it is
executed) in one of two shapes:

* a ``[layers, D, D]`` tensor, row ``i`` being decoder layer ``i``'s matrix;
* a mapping ``{index: matrix}`` or ``{"layers": {index: matrix}}``, where a matrix may also
  sit under a ``"rotation"`` key of its entry.

Matrices are kept as fp32 on the CPU. A layer's matrix must be D x D, finite and orthogonal
(every entry of R^T R within 0.015 + 0.015 |I| of the identity, the reference's acceptance
bound) before its bf16 copy goes to the device.
"""

from __future__ import annotations

from functools import lru_cache

import torch

ORTHOGONALITY_ATOL = 0.015
ORTHOGONALITY_RTOL = 0.015


def layer_index(name):
    """Decoder layer index in a module path: the integer component right after ``layers``
    (``model.layers.12.self_attn.attn`` -> 12)."""
    parts = name.split(".")
    for here, after in zip(parts, parts[1:]):
        if here == "layers" and after.isdigit():
            return int(after)
    raise ValueError(f"no decoder layer index ('layers.<i>') in module name {name!r}")


def _entries(source):
    """(index, matrix) pairs of a loaded artefact, in either accepted shape."""
    if torch.is_tensor(source):
        if source.ndim != 3:
            raise ValueError(f"a rotation tensor must be [layers, D, D], got {tuple(source.shape)}")
        return list(enumerate(source))
    if isinstance(source, dict):
        table = source["layers"] if "layers" in source else source
        if isinstance(table, dict):
            return [(key, entry.get("rotation") if isinstance(entry, dict) else entry)
                    for key, entry in table.items()]
    raise ValueError("unrecognized rotation artefact: expected a [layers, D, D] tensor or a "
                     "{layer: matrix} mapping")


@lru_cache(maxsize=4)
def load_checkpoint(path):
    """``{layer index: fp32 CPU matrix}`` of the artefact at ``path`` (cached)."""
    if not path:
        raise ValueError("no rotation artefact given: set VLLM_OSCAR_K_ROTATION_PATH and "
                         "VLLM_OSCAR_V_ROTATION_PATH to the calibrated D256 K/V rotations")
    source = torch.load(path, map_location="cpu", weights_only=True)
    table = {}
    try:
        entries = _entries(source)
    except ValueError as err:
        raise ValueError(f"{path}: {err}") from None
    for key, matrix in entries:
        if not torch.is_tensor(matrix):
            raise ValueError(f"{path}: layer {key} holds no matrix")
        table[int(key)] = matrix.detach().to(torch.float32).contiguous()
    return table


def check_rotation(matrix, dim=256, what="rotation"):
    """Raise ValueError unless ``matrix`` is a finite, orthogonal dim x dim matrix."""
    if tuple(matrix.shape) != (dim, dim):
        raise ValueError(f"{what}: expected {dim}x{dim}, got {tuple(matrix.shape)}")
    if not bool(torch.isfinite(matrix).all()):
        raise ValueError(f"{what}: contains NaN or infinite entries")
    m = matrix.to(torch.float32)
    eye = torch.eye(dim, dtype=torch.float32)
    excess = (m.T @ m - eye).abs() - (ORTHOGONALITY_ATOL + ORTHOGONALITY_RTOL * eye)
    if float(excess.max()) > 0:
        raise ValueError(f"{what}: R^T R departs from the identity by more than "
                         f"{ORTHOGONALITY_ATOL} (+{ORTHOGONALITY_RTOL} on the diagonal)")


def get_rotation(path, name, device, dim=256):
    """Validated rotation of module ``name``'s layer from the artefact at ``path``, as a
    contiguous bf16 matrix on ``device`` (reference rotations.py:36-53)."""
    index = layer_index(name)
    table = load_checkpoint(path)
    if index not in table:
        raise ValueError(f"{path} has no rotation for layer {index} ({name})")
    matrix = table[index]
    # Validation runs on the artefact's own fp32 values, before the bf16 conversion.
    check_rotation(matrix, dim, f"layer {index} rotation in {path}")
    return matrix.to(device=device, dtype=torch.bfloat16).contiguous()


def save_rotations(path, rotations):
    """Write ``{layer index: D x D matrix}`` as an artefact ``load_checkpoint`` reads."""
    layers = {int(i): {"rotation": r.detach().to(torch.float32).cpu().contiguous()}
              for i, r in rotations.items()}
    torch.save({"layers": layers}, path)
