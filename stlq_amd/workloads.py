"""Seeded synthetic workloads of the encoder benchmark configurations.

There is no dataset access, so vectors come from seeded Gaussian mixtures and the codebooks
from small seeded trainers (residual k-means, spherical k-means). Codebook training is not part
of the encoder path (the reference trains them in src/quantizer/encoder_train*.inc); these
trainers only produce realistic inputs. Everything is numpy with np.random.Generator(PCG64),
so a seed reproduces the same arrays on any machine with the same numpy.

Configurations (sizes as named by the benchmark):
  C1  100k x d128, 1024-component GMM, centres N(0,1), sigma 0.3; M=4 K=256; beam 4
  C2  1M x d128 descriptor-like: 4096-component GMM, centres N(64, 48^2), sigma 24,
      clipped to [0,255] and rounded, stored fp32; M=8 K=256; beam 16
  C3  1M x d96 unit-norm, 8192-component spherical mixture, angular spread 0.2 rad;
      spherical k-means codebooks M=8 K=256; beam 16 + 2 ICM sweeps
  C4  500k x d960, 2048 components, per-dim variance 1/(1+i/64); M=16 K=256; beam 8
  C5  streaming d128 uint8-valued (C2 generator), forced root from 65,536 root codewords,
      then 16 residual codebooks x 256; beam 32
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Workload:
    name: str
    d: int
    m: int
    K: int
    H_beam: int
    icm_iters: int = 0
    n: int = 0
    kind: str = "gauss"          # gauss | desc | sphere | decay
    n_comp: int = 1024
    seed: int = 1234
    train_n: int = 20000
    kmeans_iters: int = 8
    extra: dict = field(default_factory=dict)


CONFIGS = {
    "C1": Workload("C1", d=128, m=4, K=256, H_beam=4, n=100_000, kind="gauss", n_comp=1024, seed=11),
    "C2": Workload("C2", d=128, m=8, K=256, H_beam=16, n=1_000_000, kind="desc", n_comp=4096, seed=22),
    "C3": Workload("C3", d=96, m=8, K=256, H_beam=16, icm_iters=2, n=1_000_000, kind="sphere", n_comp=8192,
                   seed=33),
    "C4": Workload("C4", d=960, m=16, K=256, H_beam=8, n=500_000, kind="decay", n_comp=2048, seed=44,
                   train_n=10000, kmeans_iters=5),
    "C5": Workload("C5", d=128, m=17, K=256, H_beam=32, n=100_000_000, kind="desc", n_comp=4096, seed=55,
                   extra={"h0": 65536, "chunk": 4_000_000}),
}


class Mixture:
    """A seeded Gaussian-mixture generator; sample(first, count) is deterministic per row block."""

    def __init__(self, kind: str, d: int, n_comp: int, seed: int):
        self.kind, self.d, self.n_comp, self.seed = kind, d, n_comp, seed
        rng = np.random.default_rng(seed)
        if kind == "gauss":
            self.centers = rng.standard_normal((n_comp, d)).astype(np.float32)
            self.sigma = np.float32(0.3)
        elif kind == "desc":
            self.centers = (64.0 + 48.0 * rng.standard_normal((n_comp, d))).astype(np.float32)
            self.sigma = np.float32(24.0)
        elif kind == "sphere":
            c = rng.standard_normal((n_comp, d))
            self.centers = (c / np.linalg.norm(c, axis=1, keepdims=True)).astype(np.float32)
            self.sigma = np.float32(0.2 / np.sqrt(d))
        elif kind == "decay":
            self.scale = (1.0 / np.sqrt(1.0 + np.arange(d) / 64.0)).astype(np.float32)
            self.centers = (rng.standard_normal((n_comp, d)) * self.scale).astype(np.float32)
            self.sigma = np.float32(0.3)
        else:
            raise ValueError(kind)

    def _rows(self, g: int, rows: int, block: int) -> np.ndarray:
        rng = np.random.default_rng([self.seed, 7919, g // block, g % block])
        comp = rng.integers(0, self.n_comp, size=rows)
        noise = rng.standard_normal((rows, self.d), dtype=np.float32)
        if self.kind == "decay":
            noise *= self.scale
        x = self.centers[comp] + self.sigma * noise
        if self.kind == "desc":
            np.clip(np.rint(x), 0.0, 255.0, out=x)
        elif self.kind == "sphere":
            x /= np.linalg.norm(x, axis=1, keepdims=True)
        return x

    def sample(self, first: int, count: int, block: int = 65536) -> np.ndarray:
        out = np.empty((count, self.d), np.float32)
        for b0 in range(0, count, block):
            b1 = min(count, b0 + block)
            out[b0:b1] = self._rows(first + b0, b1 - b0, block)
        return out

    def sample_into(self, first: int, out: np.ndarray, executor=None, block: int = 65536) -> None:
        """sample(first, len(out)) written into `out` (float32, or uint8 for the integer-valued
        "desc" kind), its row blocks generated in parallel on `executor` when one is given."""
        count = out.shape[0]

        def one(b0):
            b1 = min(count, b0 + block)
            out[b0:b1] = self._rows(first + b0, b1 - b0, block)

        starts = range(0, count, block)
        if executor is None:
            for b0 in starts:
                one(b0)
        else:
            list(executor.map(one, starts))


def _assign(X, C, spherical):
    if spherical:
        return np.argmax(X @ C.T, axis=1)
    # argmin ||x - c||^2 = argmax (2 x.c - ||c||^2)
    return np.argmax(2.0 * (X @ C.T) - np.sum(C * C, axis=1)[None, :], axis=1)


def kmeans(X: np.ndarray, K: int, iters: int, seed: int, spherical: bool = False) -> np.ndarray:
    """Lloyd k-means (or spherical k-means) from a random-sample init; empty clusters keep
    their previous centre. float64 accumulation, float32 result."""
    rng = np.random.default_rng(seed)
    X64 = X.astype(np.float64)
    C = X64[rng.choice(X.shape[0], size=K, replace=X.shape[0] < K)].copy()
    if spherical:
        C /= np.maximum(np.linalg.norm(C, axis=1, keepdims=True), 1e-12)
    for _ in range(iters):
        lab = _assign(X64, C, spherical)
        sums = np.zeros_like(C)
        np.add.at(sums, lab, X64)
        cnt = np.bincount(lab, minlength=K).astype(np.float64)
        nz = cnt > 0
        C[nz] = sums[nz] / cnt[nz, None]
        if spherical:
            C /= np.maximum(np.linalg.norm(C, axis=1, keepdims=True), 1e-12)
    return C.astype(np.float32)


def residual_codebooks(X_train: np.ndarray, m: int, K: int, iters: int, seed: int,
                       spherical: bool = False) -> np.ndarray:
    """RVQ-style initialisation: layer l is k-means on the residual after layers < l.
    Returns C_all (m*K, d) stacked layer by layer."""
    R = X_train.astype(np.float64).copy()
    books = []
    for l in range(m):
        C = kmeans(R.astype(np.float32), K, iters, seed + 101 * l, spherical=spherical and l == 0)
        lab = _assign(R, C.astype(np.float64), spherical and l == 0)
        if spherical and l == 0:
            proj = np.sum(R * C[lab], axis=1, keepdims=True)
            R = R - proj * C[lab]
        else:
            R = R - C[lab]
        books.append(C)
    return np.concatenate(books, axis=0)


def make_codebooks(w: Workload, X_train: np.ndarray | None = None) -> np.ndarray:
    mix = Mixture(w.kind, w.d, w.n_comp, w.seed)
    if X_train is None:
        X_train = mix.sample(10_000_000, w.train_n)  # disjoint from the encoded rows
    return residual_codebooks(X_train, w.m, w.K, w.kmeans_iters, w.seed + 5, spherical=(w.kind == "sphere"))


def make_large_root(w: Workload, h0: int, n_small: int, X_train: np.ndarray | None = None):
    """Root codebook (h0 codewords = distinct training samples) and n_small residual codebooks
    trained on the residual to the nearest root."""
    mix = Mixture(w.kind, w.d, w.n_comp, w.seed)
    C0 = mix.sample(20_000_000, h0)
    if X_train is None:
        X_train = mix.sample(10_000_000, w.train_n)
    # nearest root by ||x - c||^2 for the residual codebooks
    lab = np.empty(X_train.shape[0], np.int64)
    c2 = np.sum(C0.astype(np.float64) ** 2, axis=1).astype(np.float32)
    for b0 in range(0, X_train.shape[0], 2048):
        xb = X_train[b0:b0 + 2048]
        lab[b0:b0 + 2048] = np.argmax(2.0 * (xb @ C0.T) - c2[None, :], axis=1)
    R = (X_train - C0[lab]).astype(np.float32)
    Cs = residual_codebooks(R, n_small, w.K, w.kmeans_iters, w.seed + 77)
    return C0, Cs
