"""GPU: the measurement probes read what they are credited with.

* va_probe_digest pins both forms of va_probe_read (the MBU denominator,
  src/voltattn.cu:64-78, 935-957 re-derived): over a buffer whose 16-byte
  words are all distinct, each form's XOR of the words it loaded and its load
  count must equal the host's XOR and count over exactly the bytes the probe
  credits (bytes_read), for several grids, unrolls and ragged sizes. A form
  that skips a tile, drops or repeats loads, or reads past its chunk fails
  (tests/test_probe_digest.py shows each such mistake changes the host digest).
  The buffer is padded with other words past the probed range, so a read past
  the end shows too.
* va_probe_read: a loose band only (512 MiB is partly cache-served; the bench
  probes 4 GiB). A 4 MiB buffer runs every chunked shape (some groups then get
  partial or empty chunks).
* va_probe_read_sized: the size-matched ceiling the bench reports per row: its
  time must be positive and its GB/s at most the peak plus cache headroom.
* va_probe_launch: the per-launch floor (2.5-2.9 us measured on MI355X).
"""
import numpy as np
import pytest

import voltattn_amd as va
from tests.probe_digest import pattern, xor16

pytestmark = pytest.mark.gpu

PAD = 1 << 20            # padding past the probed range: other words
SIZES = [96 << 20, (96 << 20) - 48, (1 << 20) + 16 * 3, 4096 * 33 + 16]
SHAPES = [  # (form, grid, unroll)
    (0, 1024, 4), (0, 2048, 8), (0, 8192, 8), (0, 7, 2), (0, 256 * 32, 4),
    (1, 256, 8), (1, 512, 4), (1, 256, 4), (1, 512, 8), (1, 1, 8), (1, 333, 4),
]


@pytest.fixture(scope="module")
def probe_buf():
    n = max(SIZES)
    host = pattern(n + PAD)
    host[n:] = pattern(PAD, salt=0x1234567)      # distinct words past every probed range
    buf = va.DeviceBuffer.from_array(host)
    yield buf, host
    buf.free()


@pytest.mark.parametrize("nbytes", SIZES)
@pytest.mark.parametrize("form,grid,unroll", SHAPES)
def test_probe_reads_what_it_counts(probe_buf, nbytes, form, grid, unroll):
    buf, host = probe_buf
    print(f"probe digest: form={form} grid={grid} unroll={unroll} bytes={nbytes}", flush=True)
    x, loads, credited = va.probe_digest(buf.ptr, nbytes, form, grid, unroll)
    assert credited == nbytes
    assert loads == credited // 16
    assert x == xor16(host[:credited])


def test_read_probe():
    gbps = va.probe_read(512 << 20, reps=3)
    print(f"read probe: {gbps:.0f} GB/s", flush=True)
    assert 1000.0 < gbps < 20000.0


def test_read_probe_small_buffer():
    gbps = va.probe_read(4 << 20, reps=2)
    print(f"read probe (4 MiB): {gbps:.0f} GB/s", flush=True)
    assert 0.0 < gbps < 1e6


def test_read_probe_sized():
    us, gbps = va.probe_read_sized(142606336, 1 << 30, launches=20)
    print(f"sized probe (142.6 MB): {us:.2f} us, {gbps:.0f} GB/s", flush=True)
    assert us > 0.0
    assert 500.0 < gbps < 9000.0
    us2, gbps2 = va.probe_read_sized(35651584 + 48, 1 << 30, launches=20)   # ragged last tiles
    print(f"sized probe (35.7 MB): {us2:.2f} us, {gbps2:.0f} GB/s", flush=True)
    assert 0.0 < us2 < us


def test_launch_probe():
    us = va.probe_launch(500)
    print(f"launch floor: {us:.2f} us", flush=True)
    assert 0.2 < us < 50.0


def test_probe_digest_rejects_bad_arguments(probe_buf):
    buf, _ = probe_buf
    with pytest.raises(va.VAError):
        va.probe_digest(buf.ptr, 100, 1, 256, 8)          # not a multiple of 16
    with pytest.raises(va.VAError):
        va.probe_digest(buf.ptr, 4096, 2, 256, 8)         # no form 2
    with pytest.raises(va.VAError):
        va.probe_digest(buf.ptr, 4096, 1, 256, 2)         # chunked: unroll 4 or 8
    with pytest.raises(va.VAError):
        va.probe_digest(buf.ptr + 8, 4096, 0, 256, 4)     # misaligned
