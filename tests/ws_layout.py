"""The engine workspace's layout (make_layout in astra-cuda_amd/csrc/market.hip), for
tests that compare two workspaces byte for byte.

The book state must agree exactly, but the head-size cache may know more in one
workspace than in the other: a multi-step launch caches the size of every head it
hands out as a BBO, single calls only those whose order record they hold in
registers (get_bbos reads the others from the book, so both give the same
BBOs). ``normalized`` clears the cache's flags (bit 15 of each half of the tob
word that holds a slot; an empty head, 0xFFFF, keeps its value) and its size
array, leaving everything else as it is.

The workspace starts with 256 bytes of control words (int32): the TID counter
of a book with no markets (otherwise every market keeps a copy in ``tids``) and
the count of helper wavefronts that gave up waiting.
"""
from __future__ import annotations


def _align(x: int, a: int = 256) -> int:
    return (x + a - 1) // a * a


def mask_words(L: int) -> int:
    w = 1
    while w * 64 < L:
        w *= 2
    return w


def layout(M: int, L: int, O: int, C: int) -> dict:
    """(byte offset, bytes) of each array of the workspace."""
    W = mask_words(L)
    off, out = 0, {}
    for name, nbytes in (("ctl", 256), ("masks", 2 * W * M * 8), ("next_slot", M * 4), ("tids", M * 4),
                         ("bbo", 2 * M * 4),
                         ("tob", M * 4), ("hsz", 2 * M * 4), ("levels", M * L * 8),
                         ("records", M * O * 16), ("portfolios", M * C * 8)):
        out[name] = (off, nbytes)
        off = _align(off + nbytes)
    out["total"] = (0, off)
    return out


def normalized(ws, M: int, L: int, O: int, C: int):
    """A copy of the workspace bytes (a numpy or torch uint8 array) with the
    head-size cache cleared."""
    import numpy as np
    is_np = isinstance(ws, np.ndarray)
    w = ws.copy() if is_np else ws.clone()
    lay = layout(M, L, O, C)
    o, n = lay["tob"]
    if n:
        # bit 15 of a half flags a cached size; 0xFFFF (empty) carries no flag
        if is_np:
            h = w[o:o + n].view(np.uint16)
            h[h != 0xFFFF] &= 0x7FFF
        else:
            import torch
            h = w[o:o + n].view(torch.int16)
            h.copy_(torch.where(h == -1, h, h & 0x7FFF))
    o, n = lay["hsz"]
    w[o:o + n] = 0
    return w
