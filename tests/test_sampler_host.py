"""The sampler's random stream on the host (no GPU).

``nv4_philox4x32_10`` is the Philox4x32-10 block function that
``nv4_gumbel_sample`` evaluates per 4 columns; it is pinned here against the
published known-answer vectors of Philox4x32-10 (Random123 kat_vectors:
counter/key all zeros, all ones, and the pi-digits vector).
"""
import ctypes

import pytest

from nv4 import _lib

KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


def philox(counter, key):
    c = (ctypes.c_uint32 * 4)(*counter)
    k = (ctypes.c_uint32 * 2)(*key)
    o = (ctypes.c_uint32 * 4)()
    _lib.load().nv4_philox4x32_10(c, k, o)
    return tuple(o)


@pytest.mark.parametrize("counter,key,expected", KAT)
def test_philox4x32_10_known_answers(counter, key, expected):
    assert philox(counter, key) == expected


def test_sampler_rejections():
    f = _lib.load().nv4_gumbel_sample
    P, A = ctypes.c_void_p, 0x10000
    assert f(None, 8, _lib.BF16, P(A), 2, 8, 1, 0, P(A), None) == _lib.NV4_E_NULL
    assert f(P(A), 4, _lib.BF16, P(A), 2, 8, 1, 0, P(A), None) == _lib.NV4_E_SHAPE     # row_stride < V
    assert f(P(A), 8, _lib.FP16, P(A), 2, 8, 1, 0, P(A), None) == _lib.NV4_E_DTYPE
    assert f(P(A + 1), 8, _lib.BF16, P(A), 2, 8, 1, 0, P(A), None) == _lib.NV4_E_ALIGN
    assert f(P(A + 2), 8, _lib.FP32, P(A), 2, 8, 1, 0, P(A), None) == _lib.NV4_E_ALIGN
