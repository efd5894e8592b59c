"""Cheap, reproducible full-shape inputs for a fragment -- TEST
INFRASTRUCTURE (used by make_fragment_fixtures.py and
tests/test_fragment_structure.py).

Each input takes the layout the drop-in's get_inputs builds (dtype, shape,
strides, storage offset and storage size, read from get_inputs on the meta
device, tuple inputs included) and is filled by tiling one seeded block of
2^20 + 17 normal draws over its whole storage: identical on every host and
orders of magnitude faster than drawing every element.  Integer inputs (ids,
positions, targets) take the block's values mapped into [0, 100), a valid
index for every fragment (its smallest index range is 100).
"""
from __future__ import annotations

import math

import numpy as np
import torch

BLOCK = (1 << 20) + 17


def _base(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(BLOCK, generator=g)


def _fill(meta, base):
    if isinstance(meta, (tuple, list)):
        return tuple(_fill(m, base) for m in meta)
    dt = meta.dtype
    n = meta.untyped_storage().nbytes() // meta.element_size()
    if dt.is_complex:
        real = torch.float32 if dt == torch.complex64 else torch.float64
        flat = _tile(base.to(real), 2 * n).view(dt)
    elif dt.is_floating_point:
        flat = _tile(base.to(dt), n)
    else:
        flat = _tile((base.abs() * 1000).to(torch.int64).remainder(100).to(dt), n)
    return flat.as_strided(meta.shape, meta.stride(), meta.storage_offset())


def _tile(block, n):
    reps = math.ceil(n / block.numel()) if n else 0
    return block.repeat(reps)[:n].clone() if reps else block[:0].clone()


def synth_inputs(module, seed):
    """Full-shape CPU inputs with the layout of module.get_inputs()."""
    base = _base(seed)
    return [_fill(m, base) for m in module.get_inputs(device="meta")]


SAMPLES = 48


def _tensors(x):
    return list(x) if isinstance(x, (tuple, list)) else [x]


def describe(outputs, inputs, seed):
    """Structure and sampled values of a fragment's outputs: tuple or bare;
    per output dtype, shape, strides, storage offset, its storage group
    (outputs sharing storage share a group), the input it aliases (index, or
    "i.j" inside a tuple input), and its values at 48 seeded flat positions
    (complex outputs as their real view)."""
    is_tuple = isinstance(outputs, tuple)
    outs = _tensors(outputs)
    in_storages = {}
    for i, x in enumerate(inputs):
        for j, t in enumerate(_tensors(x)):
            key = f"{i}.{j}" if isinstance(x, (tuple, list)) else f"{i}"
            in_storages.setdefault(t.untyped_storage().data_ptr(), key)
    groups, recs = {}, []
    rs = np.random.RandomState(seed)
    for t in outs:
        ptr = t.untyped_storage().data_ptr()
        groups.setdefault(ptr, len(groups))
        flat = t.detach().reshape(-1)
        if t.is_complex():
            flat = torch.view_as_real(flat).reshape(-1)
        n = flat.numel()
        pos = sorted(set([0, max(n - 1, 0)] + (rs.randint(0, n, SAMPLES - 2).tolist() if n > 2 else [])))
        vals = flat[torch.tensor(pos, dtype=torch.int64)].double().tolist() if n else []
        recs.append({
            "dtype": str(t.dtype).replace("torch.", ""), "shape": list(t.shape), "stride": list(t.stride()),
            "storage_offset": t.storage_offset(), "storage_group": groups[ptr],
            "aliases_input": in_storages.get(ptr), "positions": pos, "values": vals,
        })
    return {"tuple": is_tuple, "outputs": recs}
