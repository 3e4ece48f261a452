"""Reader of ``tests/golden/ownership_vectors.npz`` (the recorded ownership
traces) and the packing its writer uses.  Tests import this module only;
``make_ownership_vectors.py`` writes the file."""

from pathlib import Path

import numpy as np

SEEDS = range(200)
PLAN_CASES = 100_000  # direct plan cases are keyed PLAN_CASES + seed
OUT = Path(__file__).with_name("ownership_vectors.npz")

_DTYPES = ("bool", "int8", "int32", "int64", "uint8")


def pack(traces):
    """{seed: [(name, array|None)]} -> three arrays: every value flattened to
    int64 in one buffer, an index row per value (seed, dtype, ndim, dims,
    length; dtype -1 marks None) and the names."""
    data, index, names = [], [], []
    for seed, trace in traces.items():
        for name, value in trace:
            names.append(name)
            if value is None:
                index.append((seed, -1, 0, 0, 0, 0))
                continue
            v = np.asarray(value)
            dims = list(v.shape) + [0, 0]
            index.append((seed, _DTYPES.index(v.dtype.name), v.ndim, dims[0], dims[1], v.size))
            data.append(v.reshape(-1).astype(np.int64))
    return dict(data=np.concatenate(data), index=np.asarray(index, dtype=np.int64), names=np.asarray(names))


def unpack(npz):
    """Inverse of :func:`pack`: {seed: [(name, array|None)]}."""
    data, index, names = npz["data"], npz["index"], npz["names"]
    traces, at = {}, 0
    for (seed, code, ndim, d0, d1, size), name in zip(index.tolist(), names.tolist()):
        if code < 0:
            value = None
        else:
            shape = (d0, d1)[:ndim]
            value = data[at:at + size].astype(_DTYPES[code]).reshape(shape)
            at += size
        traces.setdefault(seed, []).append((str(name), value))
    return traces


def load():
    """The recorded traces, {seed: [(name, array|None)]}."""
    return unpack(np.load(OUT))
