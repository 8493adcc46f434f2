"""Closed-form index maps of the Swin block's integer work (test oracle only).

numpy restatement of the roll / window-partition / window-reverse / shift-mask
index arithmetic of the reference, plus brute-force loop versions for tiny
shapes.  The closed forms are derived from:

  * ``torch.roll`` semantics: ``roll(x, s)[h] = x[(h - s) mod H]``; the block
    rolls by ``-shift`` first (models/swin_helpers.py:402-406), so the rolled
    image row h holds original row ``(h + s0) mod H``;
  * ``window_partition`` (models/swin_helpers.py:26-51): window
    ``w = b*nW + i*(W/ws1) + j``, token ``p = t*ws0*ws1 + r*ws1 + c`` holds the
    rolled-image pixel ``(i*ws0 + r, j*ws1 + c)``;
  * ``window_reverse`` (:54-77) is the inverse permutation, and the reverse
    roll by ``+shift`` (:428-431) maps rolled row hs back to ``(hs + s0) mod H``.

Hence the fused gather (row of the window-ordered matrix <- token of x) and the
fused scatter are the same map:

    src(w, p) = (b, t, (i*ws0 + r + s0) mod H, (j*ws1 + c + s1) mod W)

and the shift mask (models/swin_helpers.py:322-397, single GPU) is

    m[w, p, q] = -100  iff  shifted and i == H/ws0 - 1 and
                            (r_p >= ws0 - s0) != (r_q >= ws0 - s0),  else 0,

with r = (p mod wa) // ws1 (the temporal part is zero for causal=False).

Pinning (tests/test_oracle_index.py): each closed form is checked bit-exact
against the brute-force loops below and against ``torch.roll`` + ``view`` /
``permute`` as the reference composes them.
"""
from __future__ import annotations

import numpy as np


def gather_rows(B: int, T: int, H: int, W: int, ws0: int, ws1: int,
                s0: int, s1: int) -> np.ndarray:
    """Flat token index (into [B,T,H,W]) for every row of the window-ordered
    matrix [B*nW*T*wa] (closed form, vectorised)."""
    nh, nw = H // ws0, W // ws1
    wa = ws0 * ws1
    b, i, j, t, r, c = np.meshgrid(np.arange(B), np.arange(nh), np.arange(nw),
                                   np.arange(T), np.arange(ws0), np.arange(ws1),
                                   indexing="ij")
    h = (i * ws0 + r + s0) % H
    w = (j * ws1 + c + s1) % W
    tok = ((b * T + t) * H + h) * W + w
    return tok.reshape(-1).astype(np.int64)


def gather_rows_bruteforce(B, T, H, W, ws0, ws1, s0, s1):
    """Pure-Python loop version of :func:`gather_rows` (tiny shapes only):
    roll by -s as torch.roll defines it, then walk the partition order."""
    rolled_src = {}
    for bb in range(B):
        for tt in range(T):
            for hh in range(H):
                for ww in range(W):
                    # torch.roll(x, -s)[h] = x[(h + s) mod H]
                    rolled_src[(bb, tt, hh, ww)] = (bb, tt, (hh + s0) % H, (ww + s1) % W)
    out = []
    for bb in range(B):
        for i in range(H // ws0):
            for j in range(W // ws1):
                for tt in range(T):
                    for r in range(ws0):
                        for c in range(ws1):
                            sb, st, sh, sw = rolled_src[(bb, tt, i * ws0 + r, j * ws1 + c)]
                            out.append(((sb * T + st) * H + sh) * W + sw)
    return np.asarray(out, dtype=np.int64)


def mask_closed_form(H: int, W: int, ws0: int, ws1: int, s0: int, s1: int,
                     T: int = 1) -> np.ndarray:
    """Additive shift mask [nW, T*wa, T*wa] (float32) from the closed form."""
    nh, nw = H // ws0, W // ws1
    wa = ws0 * ws1
    L = T * wa
    m = np.zeros((nh * nw, L, L), dtype=np.float32)
    if s0 == 0 and s1 == 0:
        return m
    p = np.arange(L)
    r = (p % wa) // ws1
    lab = (r >= ws0 - s0)
    diff = lab[:, None] != lab[None, :]
    last_band = np.arange(nh * nw) // nw == nh - 1
    m[last_band] = np.where(diff, np.float32(-100.0), np.float32(0.0))
    return m


def mask_bruteforce(H, W, ws0, ws1, s0, s1, T=1):
    """Loop version: label the un-rolled image rows as the reference does,
    partition the labels, compare every (query, key) pair."""
    nh, nw = H // ws0, W // ws1
    wa = ws0 * ws1
    L = T * wa
    label = [[0] * W for _ in range(H)]
    if s0 or s1:
        for h in range(0, H - ws0):
            for w in range(W):
                label[h][w] = 0
        for h in range(H - s0, H):
            for w in range(W):
                label[h][w] = 1
    m = np.zeros((nh * nw, L, L), dtype=np.float32)
    if not (s0 or s1):
        return m
    for i in range(nh):
        for j in range(nw):
            win = i * nw + j
            labs = []
            for t in range(T):
                for r in range(ws0):
                    for c in range(ws1):
                        labs.append(label[i * ws0 + r][j * ws1 + c])
            for pq in range(L):
                for pk in range(L):
                    if labs[pq] != labs[pk]:
                        m[win, pq, pk] = -100.0
    return m


def roll_index(H: int, W: int, s0: int, s1: int) -> np.ndarray:
    """Source flat (h, w) index of every output pixel of
    ``torch.roll(x, (s0, s1), (H-dim, W-dim))``: out[h, w] = x[(h-s0)%H, (w-s1)%W]."""
    h, w = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    return (((h - s0) % H) * W + (w - s1) % W).reshape(-1)
