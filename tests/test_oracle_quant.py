"""Oracle for the quantized matvec (attention epilogue's attn_output): ggml's
Q4_K / Q6_K / Q8_0 blocks and F32 / F16 / BF16 rows as crates/gguf/src/quant.rs
decodes and dots them.  Pinned by the reference's own tests (quant.rs:301-415,
ported with their inputs), by a float64 decoder written from the block layouts,
and by a planted nibble-order mistake.  Test infrastructure only."""
import numpy as np
import pytest

import oracle
from oracle import textbook

QK = {oracle.Q4_K: 144, oracle.Q6_K: 210, oracle.Q8_0: 34}


def f16_le(x):
    return np.array([x], np.float16).view(np.uint8)


def patterned(ty, n_blocks, mul, add, mod):  # quant.rs:303-318 / 350-357
    bb = QK[ty]
    raw = np.array([(i * mul + add) % mod for i in range(bb * n_blocks)], np.uint8)
    for b in range(n_blocks):
        off = b * bb
        if ty == oracle.Q4_K:
            raw[off:off + 2] = f16_le(0.0123)
            raw[off + 2:off + 4] = f16_le(0.0071)
        elif ty == oracle.Q6_K:
            raw[off + 208:off + 210] = f16_le(0.0123)
        else:
            raw[off:off + 2] = f16_le(0.0123)
    return raw


@pytest.mark.parametrize("ty", [oracle.Q4_K, oracle.Q6_K])
def test_kquant_dot_matches_dequant(ty):  # quant.rs:301-331, 333-336, 365-368
    raw = patterned(ty, 3, 37, 11, 251)
    n = 256 * 3
    x = np.array([((i % 17) - 8.0) * 0.05 for i in range(n)], np.float32)
    expect = float(np.dot(oracle.dequant(ty, raw, n).astype(np.float32), x))
    got = oracle.dot_row(ty, raw, x)
    assert abs(got - expect) < abs(expect) * 1e-4 + 1e-3


def test_q8_0_dot_matches_dequant():  # quant.rs:338-355
    raw = patterned(oracle.Q8_0, 3, 41, 7, 253)
    x = np.array([((i % 13) - 6.0) * 0.07 for i in range(96)], np.float32)
    expect = float(np.dot(oracle.dequant(oracle.Q8_0, raw, 96), x))
    assert abs(oracle.dot_row(oracle.Q8_0, raw, x) - expect) < abs(expect) * 1e-4 + 1e-3


def test_q8_0_decodes_signed_bytes():  # quant.rs:357-367
    blk = np.zeros(34, np.uint8)
    blk[0:2] = f16_le(0.5)
    blk[2], blk[3] = 0x80, 127
    out = oracle.dequant(oracle.Q8_0, blk, 32)
    assert out[0] == -64.0 and out[1] == 63.5


def test_q4k_six_bit_fields_read_back_as_63():  # quant.rs:375-384, through the decoder
    blk = np.zeros(144, np.uint8)
    blk[0:2] = f16_le(1.0)                  # d = 1, dmin = 0
    blk[4:16] = 0xFF                        # every 6-bit scale and min = 63
    blk[16:] = 0x11                         # every nibble 1
    np.testing.assert_array_equal(oracle.dequant(oracle.Q4_K, blk, 256), np.full(256, 63.0))


def test_q4k_zero_quants_give_negative_min():  # quant.rs:386-398
    blk = np.zeros(144, np.uint8)
    blk[0:2] = f16_le(1.0)
    blk[2:4] = f16_le(1.0)
    blk[4], blk[8] = 5, 7
    assert oracle.dequant(oracle.Q4_K, blk, 256)[0] == -7.0


def test_q6k_zero_quants_center_at_minus_32():  # quant.rs:400-409
    blk = np.zeros(210, np.uint8)
    blk[208:210] = f16_le(1.0)
    blk[192] = 2
    assert oracle.dequant(oracle.Q6_K, blk, 256)[0] == -64.0


@pytest.mark.parametrize("name", sorted(oracle.QTYPES))
def test_decoder_matches_float64_layout_reading(name):
    ty = oracle.QTYPES[name]
    w = oracle.quant_weights(ty, 4, 512, seed=3)
    got = oracle.dequant(ty, w, 4 * 512).astype(np.float64)
    ref = textbook.dequant(ty, w, 4 * 512)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7 * np.abs(ref).max())


@pytest.mark.parametrize("name", sorted(oracle.QTYPES))
def test_matvec_matches_float64(name):
    ty = oracle.QTYPES[name]
    rows, in_dim = 5, 768
    w = oracle.quant_weights(ty, rows, in_dim, seed=11)
    x = oracle.normal(12, (3, in_dim))
    y = oracle.matvec(ty, w, rows, in_dim, x)
    ref = x.astype(np.float64) @ textbook.dequant(ty, w, rows * in_dim).reshape(rows, in_dim).T
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-5 * np.abs(ref).max())


def test_planted_nibble_order_mistake_is_detected():
    w = oracle.quant_weights(oracle.Q4_K, 1, 256, seed=4)
    swapped = w.copy()
    swapped[16:] = ((w[16:] & 15) << 4) | (w[16:] >> 4)  # high and low nibbles exchanged
    x = oracle.normal(5, (256,))
    assert abs(oracle.dot_row(oracle.Q4_K, w, x) - oracle.dot_row(oracle.Q4_K, swapped, x)) > 1e-3
