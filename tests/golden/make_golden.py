"""Writes tests/golden/golden.npz: known-answer vectors for the attention path.

Inputs are the reference tests' closed-form projection and loss weights (tests/parity.rs:126-138:
qkv[i] = sin(i * 0.618034) * 1.5, w[i] = cos(i * 0.414213), f32), at the reference tests' small
shapes (tests/parity.rs:161-167, :185-204, :210-221; (b, s, h, d)), causal and not, with
scale = 1 / sqrt(d) (tests/parity.rs:80).

Expected outputs come from torch float64 autograd of an attention written here independently of
the oracle: softmax(q k^T scale + mask) v per head (the composition of tests/parity.rs:53-75),
differentiated through `sum(out * w)` by torch -- so the backward formulas restated in
oracle/composed.c are checked against autograd, not against themselves. Stored per case:
qkv, w (f32 inputs), out, lse, grad (f64).

Nothing from the reference is imported or run: its tests fix the shapes and input formulas only.
Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "golden.npz"

# (b, s, h, d)
SHAPES = [(2, 7, 3, 8), (1, 9, 2, 8), (1, 33, 2, 64), (2, 7, 3, 64), (1, 5, 1, 64)]


def closed_form(b, s, h, d):
    i = np.arange(b * s * 3 * h * d, dtype=np.float32)
    x = (np.sin(i * np.float32(0.618034)) * np.float32(1.5)).astype(np.float32)
    j = np.arange(b * s * h * d, dtype=np.float32)
    w = np.cos(j * np.float32(0.414213)).astype(np.float32)
    return x.reshape(b, s, 3 * h * d), w.reshape(b, s, h * d)


def attention64(qkv: torch.Tensor, h: int, scale: float, causal: bool):
    b, s, three_hd = qkv.shape
    hd = three_hd // 3
    d = hd // h
    q, k, v = (qkv[:, :, i * hd:(i + 1) * hd].reshape(b, s, h, d).transpose(1, 2)
               for i in range(3))
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        mask = torch.ones(s, s, dtype=torch.bool).triu(1)
        scores = scores.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    p = torch.softmax(scores, dim=-1)
    o = torch.matmul(p, v)
    return o.transpose(1, 2).reshape(b, s, hd), lse


def main():
    data = {}
    for (b, s, h, d) in SHAPES:
        for causal in (False, True):
            key = f"b{b}_s{s}_h{h}_d{d}_c{int(causal)}"
            qkv32, w32 = closed_form(b, s, h, d)
            qkv = torch.from_numpy(qkv32).double().requires_grad_(True)
            w = torch.from_numpy(w32).double()
            out, lse = attention64(qkv, h, 1.0 / d ** 0.5, causal)
            (out * w).sum().backward()
            data[f"{key}/qkv"] = qkv32
            data[f"{key}/w"] = w32
            data[f"{key}/out"] = out.detach().numpy()
            data[f"{key}/lse"] = lse.detach().numpy()
            data[f"{key}/grad"] = qkv.grad.numpy()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data) // 5} cases)")


if __name__ == "__main__":
    main()
