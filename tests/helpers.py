"""Shared helpers for the GPU parity tests: seeded inputs, building a paged
cache through the library, and reading it back in the simulation's
(b, h, tokens, d) layout for comparison with the oracle."""
from __future__ import annotations

import math

import numpy as np
import torch

NHD, HND = 0, 1


def randn16(seed, shape, scale=1.0):
    """Seeded N(0, scale^2) fp16 from numpy's PCG64 (platform independent)."""
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def outlier_keys(K, seed, n=4, factor=8.0):
    """Scale n seeded key channels by `factor` (config 2 / 5 outliers)."""
    ch = np.random.default_rng(seed).permutation(K.shape[-1])[:n]
    K = K.copy()
    K[..., ch] = (K[..., ch].astype(np.float32) * np.float32(factor)).astype(np.float16)
    return K


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def page_token(buf, layout, phys, kv, e):
    """[H, D] rows of token slot e of physical page `phys` (torch tensor)."""
    if layout == NHD:
        return buf[phys, kv, e]
    return buf[phys, kv, :, e]


def read_kv(buf, layout, pages, L):
    """Gather K and V of one sequence: returns (K, V) numpy (1, H, L, D)."""
    b = buf.cpu()
    S = b.shape[2] if layout == NHD else b.shape[3]
    ks, vs = [], []
    for t in range(L):
        p, e = divmod(t, S)
        ks.append(page_token(b, layout, pages[p], 0, e))
        vs.append(page_token(b, layout, pages[p], 1, e))
    K = torch.stack(ks, 1).numpy()[None]
    V = torch.stack(vs, 1).numpy()[None]
    return K, V


def read_filters(meta, layout, meta_pages, P):
    """(1, H, P, 2, D) numpy page filters from a metadata cache."""
    m = meta.cpu()
    S = m.shape[2] if layout == NHD else m.shape[3]
    out = []
    for p in range(P):
        mp, e = meta_pages[p // S], p % S
        out.append(torch.stack([page_token(m, layout, mp, 0, e), page_token(m, layout, mp, 1, e)], 1))
    return torch.stack(out, 1).numpy()[None]  # (1, H, P, 2, D)


def num_pages(L, S=16):
    return math.ceil(L / S)
