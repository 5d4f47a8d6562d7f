"""GPU: the measurement probes return plausible MI355X figures.

* va_probe_read (the MBU denominator, src/voltattn.cu:935-957 re-derived):
  a 512 MiB read is above the 256 MB Infinity Cache's reach only in part, so
  only a loose band is asserted (the bench probes 4 GiB); it must be positive
  and below the 8 TB/s peak plus cache headroom. A 4 MiB buffer holds fewer
  tiles than groups for three of the chunked form's four shapes (32 KiB tiles,
  or two groups per CU), which are then skipped rather than failing the probe;
  its figure is cache-served, so only that it is positive and finite is
  asserted.
* va_probe_launch (the per-launch floor the bench reports): microseconds per
  back-to-back empty launch on the decode grid; the measured 2.5-2.9 us on
  MI355X sits well inside the asserted band."""
import pytest

import voltattn_amd as va

pytestmark = pytest.mark.gpu


def test_read_probe():
    gbps = va.probe_read(512 << 20, reps=3)
    print(f"read probe: {gbps:.0f} GB/s", flush=True)
    assert 1000.0 < gbps < 20000.0


def test_launch_probe():
    us = va.probe_launch(500)
    print(f"launch floor: {us:.2f} us", flush=True)
    assert 0.2 < us < 50.0


def test_read_probe_small_buffer():
    gbps = va.probe_read(4 << 20, reps=2)
    print(f"read probe (4 MiB): {gbps:.0f} GB/s", flush=True)
    assert 0.0 < gbps < 1e6
