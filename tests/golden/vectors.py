"""Reader of tests/golden/reference_vectors.npz (written by make_golden.py from
the reference's own ATen build).

``load()`` returns {case name: {field: value}}: floating arrays as torch
tensors of the case's dtype (bf16 comes back from its stored uint16 bits),
integer arrays as torch tensors, 0-d entries as Python scalars. Nothing is
unpickled (``numpy.load(allow_pickle=False)``).
"""

from __future__ import annotations

import functools
import pathlib

import numpy as np
import torch

PATH = pathlib.Path(__file__).with_name("reference_vectors.npz")
FLOAT_FIELDS = {"q", "k", "v", "k_cache", "v_cache", "out", "k_cache_after_rows",
                "v_cache_after_rows"}
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def _tensor(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.bfloat16:
        assert a.dtype == np.uint16, a.dtype
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    t = torch.from_numpy(a.copy())
    assert t.dtype == dtype, (t.dtype, dtype)
    return t


@functools.lru_cache(maxsize=1)
def _raw() -> dict[str, np.ndarray]:
    with np.load(PATH, allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def load() -> dict[str, dict]:
    raw = _raw()
    cases: dict[str, dict] = {}
    for name in raw["cases"].tolist():
        prefix = f"{name}__"
        dtype = DTYPES[str(raw[prefix + "dtype"])]
        case: dict = {"dtype": dtype}
        for key, value in raw.items():
            if not key.startswith(prefix) or key == prefix + "dtype":
                continue
            field = key[len(prefix):]
            if field in FLOAT_FIELDS:
                case[field] = _tensor(value, dtype)
            elif value.ndim == 0:
                case[field] = value.item()
            else:
                case[field] = torch.from_numpy(value.copy())
        cases[name] = case
    return cases


def names() -> list[str]:
    return [str(n) for n in _raw()["cases"].tolist()]
