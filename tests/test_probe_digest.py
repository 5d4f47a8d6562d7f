"""CPU: the read-probe digest check has teeth.

tests/test_gpu_probes.py pins va_probe_read's two forms (src/voltattn.cu:64-78,
935-957 re-derived) by comparing each launch's digest (XOR of every 16-byte
word loaded, number of loads) with the host's XOR and count over the credited
bytes. Here the two forms' index maps are emulated on the CPU, as
voltattn_amd/csrc/va_probe.hip computes them, and plausible mistakes are
planted in the emulation: a dropped tail loop, a chunk size rounded down, a
dropped partial tile, a repeated load, an uncounted bound. Each must change the
digest, and the faithful emulation must reproduce the host's.
"""
import numpy as np
import pytest

from tests.probe_digest import pattern, xor16


def grid_stride_words(n16: int, grid: int, unroll: int, drop_tail=False, repeat_first=False):
    """Word indexes the grid-stride form loads: thread t reads t, t + stride, ...
    in rounds of `unroll` strides while the round fits, then one stride at a
    time (the tail loop)."""
    stride = grid * 256
    words = []
    t = np.arange(stride, dtype=np.int64)
    i = t.copy()
    while True:
        ok = i + (unroll - 1) * stride < n16
        if not ok.any():
            break
        for u in range(unroll):
            words.append(i[ok] + u * stride)
        i = np.where(ok, i + unroll * stride, i)
        if repeat_first:
            words.append(i[ok][:1] - unroll * stride)
            repeat_first = False
    if not drop_tail:
        while True:
            ok = i < n16
            if not ok.any():
                break
            words.append(i[ok])
            i = np.where(ok, i + stride, i)
    return np.concatenate(words) if words else np.zeros(0, np.int64)


def chunk_words(nbytes: int, grid: int, unroll: int, per_floor=False, drop_partial=False, count_all=False):
    """(word indexes loaded, loads counted) of the chunked form: group g streams
    [g*per, min(nbytes, (g+1)*per)), per = ceil(nbytes / grid) rounded up to 16,
    in tiles of 256 lanes x 16 B x unroll; loads at or past the chunk end return
    zeros and are not counted."""
    tile = 256 * 16 * unroll
    per = (nbytes // grid) // 16 * 16 if per_floor else ((nbytes + grid - 1) // grid + 15) // 16 * 16
    lane_off = np.arange(256, dtype=np.int64) * 16
    words, counted = [], 0
    for g in range(grid):
        start = g * per
        mine = 0 if start >= nbytes else min(per, nbytes - start)
        ntiles = mine // tile if drop_partial else (mine + tile - 1) // tile
        for k in range(ntiles):
            for u in range(unroll):
                off = k * tile + lane_off + u * 4096
                inb = off < mine
                words.append((start + off[inb]) // 16)
                counted += int(off.size if count_all else inb.sum())
    return (np.concatenate(words) if words else np.zeros(0, np.int64)), counted


def digest(host: np.ndarray, words: np.ndarray) -> bytes:
    w = host.view(np.uint32).reshape(-1, 4)
    return np.bitwise_xor.reduce(w[words], axis=0).astype("<u4").tobytes()


NBYTES = (1 << 20) + 16 * 3
HOST = pattern(NBYTES + 4096)


def test_pattern_is_not_degenerate():
    w = HOST.view(np.uint32).reshape(-1, 4)
    assert len({bytes(r) for r in w[:4096]}) == 4096
    assert xor16(HOST[:NBYTES]) != bytes(16)


@pytest.mark.parametrize("grid,unroll", [(7, 2), (64, 4), (512, 8)])
def test_grid_stride_emulation(grid, unroll):
    n16 = NBYTES // 16
    good = grid_stride_words(n16, grid, unroll)
    assert good.size == n16 and digest(HOST, good) == xor16(HOST[:NBYTES])
    bad = grid_stride_words(n16, grid, unroll, drop_tail=True)
    assert bad.size != n16 or digest(HOST, bad) != xor16(HOST[:NBYTES])


def test_grid_stride_repeated_load_is_seen():
    n16 = NBYTES // 16
    bad = grid_stride_words(n16, 7, 2, repeat_first=True)
    assert bad.size == n16 + 1
    assert digest(HOST, bad) != xor16(HOST[:NBYTES])


@pytest.mark.parametrize("grid,unroll", [(1, 8), (256, 8), (333, 4), (512, 4)])
def test_chunk_emulation(grid, unroll):
    expect = xor16(HOST[:NBYTES])
    words, counted = chunk_words(NBYTES, grid, unroll)
    assert counted == NBYTES // 16 and digest(HOST, words) == expect
    for mistake in ("per_floor", "drop_partial", "count_all"):
        if mistake == "per_floor" and NBYTES % (grid * 16) == 0:
            continue                     # rounding down changes nothing for this grid
        w, c = chunk_words(NBYTES, grid, unroll, **{mistake: True})
        assert c != NBYTES // 16 or digest(HOST, w) != expect, mistake


def test_half_read_is_seen():
    assert xor16(HOST[:NBYTES // 2 // 16 * 16]) != xor16(HOST[:NBYTES])
    assert xor16(HOST[:NBYTES - 16]) != xor16(HOST[:NBYTES])
