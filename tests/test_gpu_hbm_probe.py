"""Rates HBM delivers on this chip to the attention kernels' access forms (reads into registers, with
and without the non-temporal hint; direct-to-LDS copies as the dQ-from-dS kernel makes them; plain
16-byte stores; the copies also over scattered 8 and 32 KB chunks), over a buffer of the size of
config 3's dS store (4.36 GB), far beyond the caches.
tests/golden/hbm_probe.hip holds the probe. Run with -s to print the table.

The bars only check that the figures are rates of HBM (positive, below the quoted 8 TB/s peak
plus a margin for the part a 256 MB last-level cache may still hold between launches).
"""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BYTES = 4_364_000_000 // 65536 * 65536
MODES = ((0, "read, 16-byte loads"), (1, "read, 16-byte loads, non-temporal"),
         (2, "read, direct-to-LDS copies, non-temporal"), (3, "write, 16-byte stores"))


def _lib():
    lib = ctypes.CDLL(os.path.join(HERE, "golden", "libhbm_probe.so"))
    lib.hbm_probe_run.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                  ctypes.POINTER(ctypes.c_double)]
    lib.hbm_probe_run.restype = ctypes.c_int
    lib.hbm_probe_chunks.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_double)]
    lib.hbm_probe_chunks.restype = ctypes.c_int
    return lib


def rate(lib, mode, per_cu, reps=7):
    out = ctypes.c_double(0.0)
    rc = lib.hbm_probe_run(mode, BYTES, per_cu, reps, ctypes.byref(out))
    assert rc == 0, f"hbm_probe_run(mode={mode}, blocks_per_cu={per_cu}) returned {rc}"
    return out.value


def test_hbm_rates(gpu):
    lib = _lib()
    assert lib.hbm_probe_run(2, BYTES, 4, 1, ctypes.byref(ctypes.c_double())) == -1  # LDS ring: <= 2 per CU
    print(f"\nHBM rate over {BYTES / 1e9:.2f} GB, TB/s (median of 7 launches)")
    print("workgroups per CU | " + " | ".join(name for _, name in MODES))
    rows = {}
    for per_cu in (1, 2, 4, 8):
        rows[per_cu] = [rate(lib, m, per_cu) if (m != 2 or per_cu <= 2) else None for m, _ in MODES]
        print(f"{per_cu:17d} | " + " | ".join("-" if r is None else f"{r:.2f}" for r in rows[per_cu]), flush=True)
    chunks = {}
    for per_cu in (1, 2):
        for kb in (8, 32):
            out = ctypes.c_double(0.0)
            rc = lib.hbm_probe_chunks(BYTES, per_cu, kb, 7, ctypes.byref(out))
            assert rc == 0, f"hbm_probe_chunks(blocks_per_cu={per_cu}, chunk_kb={kb}) returned {rc}"
            chunks[per_cu, kb] = out.value
            print(f"read, direct-to-LDS copies, non-temporal, scattered {kb} KB chunks, {per_cu} workgroups per CU: "
                  f"{out.value:.2f}", flush=True)
    for r in [x for row in rows.values() for x in row if x is not None] + list(chunks.values()):
        assert 0.5 < r < 8.8
