"""Issue-rate table of gfx950 slots {1 MFMA 32x32x16 bf16 + V vector instructions (+1 LDS read)}.

The attention kernels run as sequences of such slots; the table converts their counted
instructions into time floors. tests/golden/issue_probe.hip holds the probe and describes the
instruction mix. Run with -s to print the table.
"""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
V_VALUES = (0, 2, 4, 6, 8, 10, 12, 14, 16, 20, 24)
MIXES = ((0, 0, "plain"), (0, 1, "exp"), (1, 0, "lds"), (1, 1, "lds+exp"))


def _lib():
    lib = ctypes.CDLL(os.path.join(HERE, "golden", "libissue_probe.so"))
    lib.issue_probe_run.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_double)]
    lib.issue_probe_run.restype = ctypes.c_int
    return lib


def slot_cycles(lib, waves, v, lds, ex, iters=500):
    out = ctypes.c_double(0.0)
    rc = lib.issue_probe_run(waves, v, lds, ex, iters, ctypes.byref(out))
    assert rc == 0, f"issue_probe_run(waves={waves}, v={v}, lds={lds}, exp={ex}) returned {rc}"
    return out.value


def test_issue_rate_table(gpu):
    lib = _lib()
    table = {}
    for waves in (1, 2):
        for lds, ex, name in MIXES:
            for v in V_VALUES:
                table[waves, name, v] = slot_cycles(lib, waves, v, lds, ex)
    print("\ncycles per SIMD slot {1 MFMA + V VALU (+1 ds_read_b128)}")
    print("  V | " + " ".join(f"{w}w {n:>8}" for w in (1, 2) for _, _, n in MIXES))
    for v in V_VALUES:
        print(f"{v:3d} | " + " ".join(f"{table[w, n, v]:11.1f}" for w in (1, 2) for _, _, n in MIXES))
    for waves in (1, 2):
        # a lone 32x32x16 bf16 product occupies the matrix core for 32 cycles
        assert 30.0 <= table[waves, "plain", 0] <= 36.0
    # two waves per SIMD hide a few vector instructions per product completely ...
    assert table[2, "plain", 4] <= 36.0
    # ... and a long vector slice makes the slot vector-bound (each instruction takes > 2 cycles)
    assert table[2, "plain", 24] >= 24 * 2.5
    for waves in (1, 2):
        for _, _, name in MIXES:
            seq = [table[waves, name, v] for v in V_VALUES]
            assert all(b >= a - 2.0 for a, b in zip(seq, seq[1:])), (waves, name, seq)
