"""Deterministic synthetic [B, V] fp32 logits for the benchmark configs.

Each generator draws from numpy's PCG64 with a fixed seed, so the same
buffer is produced on every machine; the GPU run and the CPU oracle are fed
the identical array.  Row RNG seeds follow each config's description.
"""
import dataclasses
from typing import Callable, Dict, List

import numpy as np


@dataclasses.dataclass
class Workload:
    name: str
    B: int
    V: int
    temperature: float
    top_p: float
    seeds: List[int]
    greedy_pass: bool
    make: Callable[[int], np.ndarray]  # rows -> [rows, V] float32
    description: str


def _normal(seed, B, V, sigma):
    g = np.random.Generator(np.random.PCG64(seed))
    return (g.standard_normal((B, V), dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def rotation(x: np.ndarray, i: int) -> np.ndarray:
    """The i-th of the benchmark's rotated batches: rows permuted (PCG64 seed
    i) and every row rolled by 997*i columns; rotation 0 is x itself.  Same
    distribution, distinct rows and addresses."""
    if i == 0:
        return x
    perm = np.random.Generator(np.random.PCG64(i)).permutation(x.shape[0])
    return np.ascontiguousarray(np.roll(x[perm], 997 * i, axis=1))


def headline(B=256, V=50257):
    return _normal(7, B, V, 3.0)


def c1(B=1, V=50257):
    return _normal(7, B, V, 3.0)


def c2(B=64, V=50257):
    g = np.random.Generator(np.random.PCG64(2))
    x = g.standard_normal((B, V), dtype=np.float32)
    for r in range(B):
        n = int(g.integers(1, 6))
        pos = g.choice(V, size=n, replace=False)
        x[r, pos] += g.uniform(8.0, 15.0, size=n).astype(np.float32)
    return x


def c3(B=256, V=49152):
    g = np.random.Generator(np.random.PCG64(3))
    ranks = np.arange(1, V + 1, dtype=np.float64)
    base = -1.1 * np.log(ranks)
    x = np.empty((B, V), dtype=np.float32)
    for r in range(B):
        perm = g.permutation(V)
        x[r] = (base[perm] + g.normal(0.0, 0.5, size=V)).astype(np.float32)
    return x


def c4(B=512, V=128256):
    g = np.random.Generator(np.random.PCG64(4))
    x = (g.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    for r in range(0, B, 10):
        m = x[r].max()
        extra = int(g.integers(1, 4))
        pos = g.choice(V, size=extra, replace=False)
        x[r, pos] = m
    return x


def c5(B=1024, V=50257):
    g = np.random.Generator(np.random.PCG64(5))
    return g.uniform(-0.5, 0.5, size=(B, V)).astype(np.float32)


WORKLOADS: Dict[str, Workload] = {
    "headline": Workload("headline", 256, 50257, 0.8, 0.9, list(range(256)), False,
                         lambda B: headline(B), "B=256 V=50257 N(0,3^2) seed 7, T=0.8 top-p=0.9"),
    "c1": Workload("c1", 1, 50257, 0.8, 0.9, [7], True, lambda B: c1(B),
                   "B=1 V=50257 N(0,3^2) seed 7; greedy and T=0.8 top-p=0.9 seed 7"),
    "c2": Workload("c2", 64, 50257, 1.0, 0.95, list(range(64)), False, lambda B: c2(B),
                   "B=64 V=50257 N(0,1) + 1-5 peaks +U[8,15); T=1.0 top-p=0.95 seeds 0..63"),
    "c3": Workload("c3", 256, 49152, 0.7, 0.9, list(range(256)), True, lambda B: c3(B),
                   "B=256 V=49152 Zipf -1.1 ln(rank)+N(0,0.5^2); T=0.7 top-p=0.9 + greedy"),
    "c4": Workload("c4", 512, 128256, 0.8, 0.9, list(range(512)), True, lambda B: c4(B),
                   "B=512 V=128256 N(0,2^2), 10% rows with tied maxima; greedy + T=0.8 top-p=0.9"),
    "c5": Workload("c5", 1024, 50257, 1.3, 0.99, list(range(1000, 2024)), False, lambda B: c5(B),
                   "B=1024 V=50257 U(-0.5,0.5); T=1.3 top-p=0.99 seeds 1000..2023"),
}
