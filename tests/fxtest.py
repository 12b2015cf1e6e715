"""Shared helpers of the tests: the oracle-side weight mappings and small utilities.

Only tests import this (it imports the oracle)."""
import numpy as np

from oracle import oracle as O
from fleet import pack_weights as P

SEED = 20261201


def rng_bf16(rng, shape, scale=1.0):
    return O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def cpu_gen(seed, stream, n, scale, offset):
    return O.gen_normal_bf16(seed, stream, n, scale, offset=offset)


class SeededCpuWeights(dict):
    """Packed weights regenerated on the CPU from the seed (oracle generator), lazily per key and
    per expert slab; the mapping the oracle's model.decode_step reads."""

    def __init__(self, dims, seed, layers, head=True):
        super().__init__()
        self.layout = P.seeded_layout(dims, layers, head)
        self.seed = seed
        self.dims = dims
        self._experts = {}

    def __missing__(self, key):
        v = P.materialize(self.layout[key], self.seed, cpu_gen)
        self[key] = v
        return v

    def expert(self, key, e):
        k = (key, e)
        if k not in self._experts:
            pt = self.layout[key]
            per = int(np.prod(pt.shape[1:]))
            self._experts[k] = P.materialize(pt, self.seed, cpu_gen, P.expert_segments(pt, e, per), pt.shape[1:])
        return self._experts[k]


class GpuWeights(dict):
    """Packed weights downloaded from the device buffers (large tensors, one expert slab at a time)."""

    def __init__(self, bufs):
        super().__init__()
        self.bufs = bufs
        self._experts = {}

    def __missing__(self, key):
        v = self.bufs[key].download()
        self[key] = v
        return v

    def expert(self, key, e):
        k = (key, e)
        if k not in self._experts:
            b = self.bufs[key]
            per = int(np.prod(b.shape[1:]))
            self._experts[k] = b.download_range(e * per, per).reshape(b.shape[1:])
        return self._experts[k]


def mismatch(a, b):
    """Count of differing elements (bit patterns for uint arrays)."""
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype == np.float32:
        return int(np.count_nonzero(a.view(np.uint32) != b.view(np.uint32)))
    return int(np.count_nonzero(a != b))
