"""The bf16 GELU table of the generator (ethos_amd/csrc/gelu_bf16_lut.inc, written by
gelu_lut.py) and the closed forms used outside it reproduce the oracle's
RN_bf16(GELU(x)) for every bf16 input x."""
import os
import re
import sys

import numpy as np

from oracle import oracle as O

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ethos_amd", "csrc")
sys.path.insert(0, CSRC)
import gelu_lut  # noqa: E402


def _inc_table():
    txt = open(os.path.join(CSRC, "gelu_bf16_lut.inc")).read()
    return np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{4})", txt)], dtype=np.uint16)


def test_include_is_generated_table():
    t = _inc_table()
    assert len(t) == 3328
    assert np.array_equal(t, np.array(gelu_lut.table(), dtype=np.uint16))


def test_table_and_closed_forms_cover_every_bf16_input():
    bits = np.arange(65536, dtype=np.uint32)
    x = O.bf16_bits_to_f32(bits.astype(np.uint16))
    with np.errstate(invalid="ignore"):
        ref = O.f32_to_bf16_bits(O.round_T(O.gelu64(x.astype(np.float64)), "bf16"))
        half = O.f32_to_bf16_bits((x * np.float32(0.5)).astype(np.float32))
    t = _inc_table()
    a = (bits & 0x7FFF).astype(np.int64)
    neg = (bits >> 15).astype(np.int64)
    got = t[np.clip(a - 0x3A80 + 1536 * neg, 0, 3327)].copy()
    small = a < 0x3A80
    big_pos = (neg == 0) & (a >= 0x4080)
    big_neg = (neg == 1) & (a >= 0x4180)
    got[big_pos] = bits[big_pos]
    got[big_neg] = np.where(a[big_neg] >= 0x7F80, 0xFFC0, 0x8000)
    got[small] = half[small]
    nan_ref = np.isnan(O.bf16_bits_to_f32(ref))
    nan_got = np.isnan(O.bf16_bits_to_f32(got))
    assert np.array_equal(nan_got, nan_ref)
    assert np.array_equal(got[~nan_ref], ref[~nan_ref])
    # the table is not trivially the identity / zero anywhere it is used
    assert np.mean(t[:1536] == np.arange(0x3A80, 0x3A80 + 1536)) < 0.5
