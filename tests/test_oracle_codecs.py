"""fp16 codecs of the oracle and the product compiler, no GPU.

* binary16 -> binary32 (kernel.cu:43-47 uses __half2float): all 65,536 patterns against
  numpy's float16, bit for bit (NaNs compared as NaN);
* binary32 -> binary16 round-to-nearest-even: against numpy's float16 cast on every
  251st float32 pattern plus the neighbourhoods of all half-way points;
* the reference's truncating float_to_half (projects/voxel-dag/src/compiler.cpp:542-560):
  bit patterns derived by hand from its integer steps.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle


def test_half_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.half_to_float(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_half_encode_rne_matches_numpy():
    pats = np.arange(0, 2**32, 251, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = oracle.float_to_half(vals)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7C00) == 0x7C00).all() and ((got[nan] & 0x3FF) != 0).all()


def test_half_encode_rne_halfway_points():
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in binary32
    around = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))])
    around = np.concatenate([around, -around])
    with np.errstate(over="ignore"):
        want = around.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.float_to_half(around), want)


@pytest.mark.parametrize("value,bits", [
    (0.0, 0x7C00),                  # biased exponent wraps below 0 -> "e > 30" -> +inf
    (1e-5, 0x7C00),                 # below 2^-15: same wrap
    (1.0, 0x3C00),
    (0.5, 0x3800),
    (1.0 + 2.0 ** -11, 0x3C00),     # exact tie: truncates
    (1.0 + 3 * 2.0 ** -12, 0x3C00),  # RNE would round up to 0x3C01; the quirk truncates
    (1.5 * 2.0 ** -15, 0x0300),     # exponent field 112 -> the e == 0 branch: (m|2^23)>>1>>13
    (65504.0, 0x7BFF),
    (65536.0, 0x7C00),              # e = 31 > 30 -> inf
    (-2.0, 0xC000),
])
def test_reference_quirk_encoder(value, bits):
    assert int(oracle.float_to_half(np.array([value], np.float32), quirk=True)[0]) == bits


def test_quirk_differs_from_rne_where_documented():
    assert int(oracle.float_to_half(np.array([1.0 + 3 * 2.0 ** -12], np.float32))[0]) == 0x3C01
    assert int(oracle.float_to_half(np.array([0.0], np.float32))[0]) == 0x0000
