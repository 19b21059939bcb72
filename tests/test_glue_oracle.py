"""Pins the oracle of the dX handoff castFloatToBfloat (elementwise.metal:19-28) without a GPU:
known answers for round-to-nearest-even (ties to even both ways, carries into the exponent,
overflow to infinity, subnormals, signed zero) and, on random and special inputs, agreement with
torch's own float32 -> bfloat16 conversion on the CPU (a library routine that rounds to nearest
even)."""
import numpy as np
import torch

import oracle as O


def bits(vals):
    return np.array(vals, dtype=np.uint32).view(np.float32)


def test_known_answers():
    x = bits([0x3F800000,   # 1.0
              0x3F808000,   # 1 + 2^-8: a tie, rounds down to the even 0x3F80
              0x3F818000,   # 1 + 3*2^-8: a tie, rounds up to the even 0x3F82
              0x3F808001,   # just above the tie: up
              0x3F7FFFFF,   # carry into the exponent: 1.0
              0x7F7FFFFF,   # largest finite: overflows to +inf
              0xFF7FFFFF,   # to -inf
              0x7F800000, 0xFF800000,  # infinities stay
              0x80000000, 0x00000000,  # signed zeros
              0x00018000,   # subnormal tie between 0x0001 and 0x0002: up to the even 0x0002
              0x7F800001,   # signalling NaN: quiet NaN, same sign
              0xFFC12345])  # quiet negative NaN keeps sign and top payload bits
    want = [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x3F80, 0x7F80, 0xFF80, 0x7F80, 0xFF80, 0x8000, 0x0000, 0x0002,
            0x7FC0, 0xFFC1]
    assert O.castFloatToBfloat(x).tolist() == want


def test_matches_torch_conversion():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32),
        (rng.standard_normal(10_000) * 1e-40).astype(np.float32),          # subnormals
        rng.integers(0, 2 ** 32, size=100_000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # every class
    ])
    got = O.castFloatToBfloat(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    g = got[nan]
    assert ((g & 0x7F80) == 0x7F80).all() and ((g & 0x7F) != 0).all()  # NaN stays NaN
    assert np.array_equal(g >> 15, (x[nan].view(np.uint32) >> 31).astype(np.uint16))  # sign kept


def test_planted_truncation_is_caught():
    """Truncation instead of rounding (a plausible mistake) fails the known answers."""
    x = bits([0x3F808001, 0x3F7FFFFF])
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert trunc.tolist() != O.castFloatToBfloat(x).tolist()
