"""Pin the CPU oracle (oracle/oracle.c) before trusting it.

Checks, per function: the reference's own known-answer fixtures (tests/test_phase2a.cpp of the
reference, transcribed in tests/golden/ref_kat.json), bitwise equality with the reference's own
code compiled from its sources (golden vectors in tests/golden/ref_random.npz, and live when
oracle/_ref/libref.so is present), IEEE/numpy for binary16, GGML invariants for Q8_K, and a
byte-centric restatement of the block layouts for single-hot fixtures.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import hexbytes
from oracle_amd import synth

ORC_INVALID_ARGUMENT, ORC_OUT_OF_RANGE, ORC_OVERFLOW, ORC_RUNTIME_ERROR = -1, -2, -3, -4


def f16row(bits):
    return np.array(bits, dtype="<u2").view(np.uint8)


# ---------------------------------------------------------------- binary16 / bfloat16

def test_f16_known_answers(kat):
    for bits, want in kat["f16"]:
        assert oracle.f16_to_f32(bits) == want
    sp = kat["f16_special"]
    assert math.isinf(oracle.f16_to_f32(sp["inf"]))
    assert math.isnan(oracle.f16_to_f32(sp["nan"]))
    assert math.copysign(1.0, oracle.f16_to_f32(sp["neg_zero"])) == -1.0


def test_f16_all_inputs_match_reference_and_ieee(golden):
    bits = golden["f16_all_bits"]
    dec = oracle.decode_row(1, 65536, bits.view(np.uint8))
    assert np.array_equal(dec.view(np.uint32), golden["f16_all_decoded_bits"])
    ieee = bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ieee)
    assert np.array_equal(dec[finite].view(np.uint32), ieee[finite].view(np.uint32))
    # NaN payloads survive: mantissa bits shifted into place, never quieted
    nan_bits = bits[~finite]
    assert np.array_equal(dec[~finite].view(np.uint32) & 0x7FFFFF, (nan_bits.astype(np.uint32) & 0x3FF) << 13)


def test_bf16_known_answers_and_rows(kat, golden):
    for bits, want in kat["bf16"]:
        assert oracle.lib().orc_bf16_to_f32(bits) == want
    for key, t in (("f16_row", 1), ("bf16_row", 30)):
        got = oracle.decode_row(t, 4, f16row(kat[key]["bits"]))
        assert got.tolist() == kat[key]["expected"]
    dec = oracle.decode_row(30, 4096, golden["bf16_sample_bits"].view(np.uint8))
    assert np.array_equal(dec.view(np.uint32), golden["bf16_sample_decoded_bits"])


# ---------------------------------------------------------------- reference known answers

def test_q5_k_known_answers(kat):
    blk = hexbytes(kat["q5_k"]["block"])
    dec = oracle.decode_row(13, 256, blk)
    for g in range(4):
        assert np.all(dec[g * 64:g * 64 + 32] == kat["q5_k"]["low"])
        assert np.all(dec[g * 64 + 32:g * 64 + 64] == kat["q5_k"]["high"])
    assert oracle.storage_dot(13, 256, blk, np.ones(256, np.float32)) == kat["q5_k"]["dot_ones"]
    two = np.concatenate([blk, blk])
    assert oracle.storage_dot(13, 512, two, np.ones(512, np.float32)) == kat["q5_k"]["dot_ones_two_blocks"]
    rows = np.concatenate([hexbytes(r) for r in kat["q5_k_matvec"]["rows"]])
    y = oracle.storage_matvec(13, 2, 256, rows, np.ones(256, np.float32))
    assert y.tolist() == kat["q5_k_matvec"]["expected"]


def test_q6_k_known_answers(kat):
    blk = hexbytes(kat["q6_k"]["block"])
    dec = oracle.decode_row(14, 256, blk)
    for half in range(2):
        assert np.all(dec[half * 128:half * 128 + 64] == kat["q6_k"]["lower"])
        assert np.all(dec[half * 128 + 64:half * 128 + 128] == kat["q6_k"]["upper"])
    assert oracle.storage_dot(14, 256, blk, np.ones(256, np.float32)) == kat["q6_k"]["dot_ones"]


def test_q8_0_known_answers(kat):
    blk = hexbytes(kat["q8_0"]["block"])
    assert oracle.decode_row(8, 32, blk).tolist() == kat["q8_0"]["expected"]
    assert oracle.storage_dot(8, 32, blk, np.ones(32, np.float32)) == kat["q8_0"]["dot_ones"]
    two = oracle.decode_row(8, 64, hexbytes(kat["q8_0_two_blocks"]["blocks"]))
    assert (two[3], two[32], two[63]) == (kat["q8_0_two_blocks"]["at3"], kat["q8_0_two_blocks"]["at32"],
                                          kat["q8_0_two_blocks"]["at63"])
    rows = np.concatenate([hexbytes(r) for r in kat["q8_0_matvec"]["rows"]])
    assert oracle.storage_matvec(8, 2, 32, rows, np.ones(32, np.float32)).tolist() == kat["q8_0_matvec"]["expected"]


# ---------------------------------------------------------------- reference on random rows (golden)

@pytest.mark.parametrize("name", ["q5_k", "q6_k", "q8_0", "q5_k_raw", "q6_k_raw", "q8_0_raw"])
def test_random_rows_bitwise_equal_reference(golden, name):
    t = int(golden[f"{name}_type"][0])
    data = golden[f"{name}_bytes"]
    rows, cols = golden[f"{name}_decoded_bits"].shape
    dec = oracle.decode_matrix(t, cols, rows, data)
    assert np.array_equal(dec.view(np.uint32), golden[f"{name}_decoded_bits"])
    y = oracle.storage_matvec(t, rows, cols, data, golden["x"])
    assert np.array_equal(y.view(np.uint32), golden[f"{name}_matvec_bits"])


def test_q4_k_equals_reference_q5_k_without_fifth_bits(golden):
    data = golden["q4_k_bytes"]
    rows, cols = golden["q4_k_decoded_bits"].shape
    dec = oracle.decode_matrix(12, cols, rows, data)
    assert np.array_equal(dec.view(np.uint32), golden["q4_k_decoded_bits"])
    y = oracle.storage_matvec(12, rows, cols, data, golden["x"])
    assert np.array_equal(y.view(np.uint32), golden["q4_k_matvec_bits"])


# ---------------------------------------------------------------- Q4_K derived fixtures

def test_q4_k_derived_known_answers(kat):
    # the reference's Q5_K header (d=0.5, dmin=0.25, every sc=2, m=3) on a Q4_K block
    hdr = hexbytes(kat["q5_k"]["block"])[:16]
    blk = np.concatenate([hdr, np.full(128, 0x21, np.uint8)])
    dec = oracle.decode_row(12, 256, blk)
    for g in range(4):
        assert np.all(dec[g * 64:g * 64 + 32] == 0.25)       # 0.5*2*1 - 0.25*3
        assert np.all(dec[g * 64 + 32:g * 64 + 64] == 1.25)  # 0.5*2*2 - 0.25*3
    assert oracle.storage_dot(12, 256, blk, np.ones(256, np.float32)) == 192.0
    zero = np.concatenate([hdr, np.zeros(128, np.uint8)])
    assert np.all(oracle.decode_row(12, 256, zero) == -0.75)
    assert oracle.storage_dot(12, 256, zero, np.ones(256, np.float32)) == -192.0


def _scale_pair_block(j, s, m):
    sc = np.zeros((1, 8), np.uint8)
    mn = np.zeros((1, 8), np.uint8)
    sc[0, j], mn[0, j] = s, m
    return synth.pack_scale_min_k4(sc, mn)[0]


@pytest.mark.parametrize("j", range(8))
def test_q4_k_single_hot_scale_pairs(j):
    # d = 1, dmin = 1 (0x3C00), one (scale, min) pair set; every 4-bit quant = 5
    s, m = 37 + j, 50 - j  # exercise both 6-bit halves
    blk = np.concatenate([f16row([0x3C00, 0x3C00]), _scale_pair_block(j, s, m), np.full(128, 0x55, np.uint8)])
    dec = oracle.decode_row(12, 256, blk)
    for sub in range(8):
        want = (s * 5 - m) if sub == j else 0.0
        assert np.all(dec[sub * 32:(sub + 1) * 32] == want), (j, sub)


def _q6_bytecentric(blk):
    """GGML's Q6_K layout read byte by byte: for half h and l in 0..31, ql[64h+l] carries the
    low nibbles of y[128h+l] (bits 0-3) and y[128h+l+64] (bits 4-7); ql[64h+l+32] those of
    y[128h+l+32] and y[128h+l+96]; qh[32h+l] bit pairs 0,2,4,6 give the high bits of y[128h+l],
    +32, +64, +96; the scale of y[128h + 16*i + r] is sc[8h + i]."""
    ql, qh, sc = blk[:128], blk[128:192], blk[192:208].view(np.int8)
    d = float(np.frombuffer(blk[208:210].tobytes(), "<f2")[0])
    y = np.zeros(256)
    for h in range(2):
        for l in range(32):
            a, b, c = ql[64 * h + l], ql[64 * h + l + 32], qh[32 * h + l]
            q = [(a & 15) | ((c & 3) << 4), (b & 15) | (((c >> 2) & 3) << 4),
                 (a >> 4) | (((c >> 4) & 3) << 4), (b >> 4) | (((c >> 6) & 3) << 4)]
            for s in range(4):
                i = 128 * h + 32 * s + l
                y[i] = d * int(sc[8 * h + i % 128 // 16]) * (int(q[s]) - 32)
    return y


def test_q6_k_single_hot_against_bytecentric_layout():
    rng = np.random.default_rng(7)
    base = np.zeros(210, np.uint8)
    base[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    base[208:210] = f16row([0x3C00])
    cases = [base.copy()]
    for pos in list(range(0, 192, 7)) + [191]:
        for val in (0x01, 0x10, 0x40):
            b = base.copy()
            b[pos] = val
            cases.append(b)
    for _ in range(20):
        b = np.frombuffer(rng.bytes(210), np.uint8).copy()
        b[208:210] = f16row([0x3800])
        cases.append(b)
    for b in cases:
        assert np.array_equal(oracle.decode_row(14, 256, b).astype(np.float64), _q6_bytecentric(b))


# ---------------------------------------------------------------- Q8_K

def _q8k_fields(blk):
    d = np.frombuffer(blk[:4].tobytes(), "<f4")[0]
    q = blk[4:260].view(np.int8).astype(np.int32)
    bs = np.frombuffer(blk[260:292].tobytes(), "<i2").astype(np.int32)
    return d, q, bs


def test_q8k_hand_known_answers():
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    d, q, bs = _q8k_fields(oracle.quantize_q8k(x))
    assert d == np.float32(1.0) / np.float32(-127.0) and q[0] == -127 and not q[1:].any()
    assert bs[0] == -127 and not bs[1:].any()
    x = np.zeros(256, np.float32)
    x[0], x[1] = -2.0, 2.0  # tie on |x|: the first index decides max = -2, iscale = 63.5
    d, q, bs = _q8k_fields(oracle.quantize_q8k(x))
    assert (q[0], q[1]) == (-127, 127) and d == np.float32(1.0) / np.float32(63.5)
    x[0], x[1] = 2.0, -2.0
    d, q, _ = _q8k_fields(oracle.quantize_q8k(x))
    assert (q[0], q[1]) == (-127, 127) and d < 0
    d, q, bs = _q8k_fields(oracle.quantize_q8k(np.zeros(256, np.float32)))
    assert d == 0 and not q.any() and not bs.any()
    # round-half-even at iscale*x = 0.5 and 1.5: x = [-127, 0.5, 1.5, 2.5] -> iscale = 1
    x = np.zeros(256, np.float32)
    x[:4] = [-127.0, 0.5, 1.5, 2.5]
    _, q, _ = _q8k_fields(oracle.quantize_q8k(x))
    assert q[:4].tolist() == [-127, 0, 2, 2]


def test_q8k_invariants_on_random_blocks():
    rng = np.random.default_rng(3)
    for scale in (1e-30, 1e-3, 1.0, 1e4, 1e30):
        x = (rng.standard_normal(256 * 16) * scale).astype(np.float32)
        x[300:310] = 0.0
        blocks = oracle.quantize_q8k(x).reshape(16, 292)
        for b in range(16):
            xb = x[b * 256:(b + 1) * 256]
            d, q, bs = _q8k_fields(blocks[b])
            assert np.all(np.abs(q) <= 127)
            first = int(np.argmax(np.abs(xb)))
            assert q[first] == -127
            assert (d < 0) == (xb[first] > 0)
            assert np.array_equal(bs, q.reshape(16, 16).sum(1))
            err = np.abs(d.astype(np.float64) * q - xb.astype(np.float64))
            assert np.all(err <= abs(float(d)) * (0.5 + 1e-6) + 1e-45)
    back = oracle.dequantize_q8k(oracle.quantize_q8k(np.ones(256, np.float32)), 256)
    assert np.allclose(back, 1.0, atol=1 / 127)


# ---------------------------------------------------------------- integer Q x Q8_K dots

def _exact_kquant_dot(t, wrow, q8blk):
    """Exact rational value of GGML's integer formula with Python ints/floats (brute force)."""
    dx, q8, bs = _q8k_fields(q8blk)
    if t == 14:
        d = float(np.frombuffer(wrow[208:210].tobytes(), "<f2")[0])
        dec = oracle.decode_row(14, 256, wrow) / np.float32(d) if d else np.zeros(256)
        # decoded / d = sc*(q-32) exactly (both small integers)
        ints = np.rint(dec).astype(np.int64)
        return d * float(dx) * int((ints * q8).sum())
    d = float(np.frombuffer(wrow[0:2].tobytes(), "<f2")[0])
    dmin = float(np.frombuffer(wrow[2:4].tobytes(), "<f2")[0])
    total_sc, total_m = 0, 0
    for j in range(8):
        s, m = [int(v) for v in _unpack(j, wrow[4:16])]
        g, hi = j // 2, j % 2
        qs = wrow[16 + 32 * g:16 + 32 * g + 32]
        q4 = (qs >> 4) if hi else (qs & 15)
        total_sc += s * int((q4.astype(np.int64) * q8[64 * g + 32 * hi:64 * g + 32 * hi + 32]).sum())
        total_m += m * int(bs[2 * j] + bs[2 * j + 1])
    return d * float(dx) * total_sc - dmin * float(dx) * total_m


def _unpack(j, p):
    p = [int(v) for v in p]
    if j < 4:
        return p[j] & 63, p[j + 4] & 63
    return (p[j + 4] & 15) | ((p[j - 4] >> 6) << 4), (p[j + 4] >> 4) | ((p[j] >> 6) << 4)


@pytest.mark.parametrize("t", [12, 14])
def test_integer_dot_matches_float_dot(t):
    rng = np.random.default_rng(11 + t)
    rows, cols = 8, 1024
    data = synth.weights(t, rng, rows, cols).reshape(rows, -1)
    x = rng.standard_normal(cols).astype(np.float32)
    q8 = oracle.quantize_q8k(x)
    xhat = oracle.dequantize_q8k(q8, cols)
    for r in range(rows):
        idot = oracle.vec_dot_q8k(t, cols, data[r], q8)
        fdot = oracle.storage_dot(t, cols, data[r], xhat)
        _, ab = oracle.matvec_stats(t, 1, cols, data[r], xhat, threads=1)
        assert abs(idot - fdot) <= 1e-5 * ab[0]
        exact = sum(_exact_kquant_dot(t, data[r].reshape(-1, {12: 144, 14: 210}[t])[b],
                                      q8.reshape(-1, 292)[b]) for b in range(cols // 256))
        assert abs(idot - exact) <= 1e-6 * ab[0]


# ---------------------------------------------------------------- registry and error paths

def test_registry_matches_reference():
    if not oracle.ref_available():
        pytest.skip("compiled reference not built")
    import ctypes as C
    for t in range(50):
        be, bpb, q = C.c_uint64(), C.c_uint64(), C.c_int()
        name = C.create_string_buffer(64)
        rrc = oracle.ref().ref_type_layout(t, C.byref(be), C.byref(bpb), C.byref(q), name, 64)
        obe, obpb, oq = C.c_uint64(), C.c_uint64(), C.c_int()
        oname = C.c_char_p()
        orc = oracle.lib().orc_type_layout(t, C.byref(obe), C.byref(obpb), C.byref(oq), C.byref(oname))
        assert (rrc == 0) == (orc == 0), t
        if rrc == 0:
            assert (be.value, bpb.value, q.value, name.value) == (obe.value, obpb.value, oq.value, oname.value)
        for n in (0, 1, 32, 256, 255, 4096):
            r_out, o_out = C.c_uint64(), C.c_uint64()
            a = oracle.ref().ref_row_byte_size(n, t, C.byref(r_out))
            b = oracle.lib().orc_row_byte_size(n, t, C.byref(o_out))
            assert a == b, (t, n)
            if a == 0:
                assert r_out.value == o_out.value


def test_error_kinds_match_reference():
    if not oracle.ref_available():
        pytest.skip("compiled reference not built")
    import ctypes as C
    q5 = np.zeros(176, np.uint8)
    x = np.ones(256, np.float32)
    y = np.zeros(4, np.float32)
    cases = [
        (13, 256, q5[:2]),        # truncated row
        (0, 1, q5[:2]),           # f32 row of wrong size
        (2, 32, np.zeros(18, np.uint8)),  # registered but not decodable (q4_0)
        (8, 17, np.zeros(34, np.uint8)),  # ragged q8_0 row
        (99, 256, q5),            # unregistered type
        (13, 0, q5),              # zero elements
    ]
    for t, n, b in cases:
        rrc = oracle.ref().ref_decode_row(t, n, b.ctypes.data, b.nbytes, y.ctypes.data, 4 if n == 0 else n)
        orc = oracle.check_row(t, n, b.nbytes)
        assert rrc == orc, (t, n, rrc, orc)
    # matvec: zero dims, vector length mismatch, matrix byte size mismatch
    m = np.zeros(352, np.uint8)
    assert oracle.ref().ref_storage_matvec(13, 0, 256, m.ctypes.data, 352, x.ctypes.data, 256, y.ctypes.data, 0) \
        == ORC_INVALID_ARGUMENT
    assert oracle.ref().ref_storage_matvec(13, 2, 256, m.ctypes.data, 351, x.ctypes.data, 256, y.ctypes.data, 2) \
        == ORC_INVALID_ARGUMENT
    out = np.zeros(2, np.float32)
    assert oracle.lib().orc_storage_matvec(13, 0, 256, m.ctypes.data, 352, x.ctypes.data, out.ctypes.data) \
        == ORC_INVALID_ARGUMENT
    assert oracle.lib().orc_storage_matvec(13, 2, 256, m.ctypes.data, 351, x.ctypes.data, out.ctypes.data) \
        == ORC_INVALID_ARGUMENT
    # Q4_K: the reference's decoder whitelist rejects it; the restatement (and the drop-in) add it
    q4 = np.zeros(144, np.uint8)
    assert oracle.ref().ref_decode_row(12, 256, q4.ctypes.data, 144, y.ctypes.data, 256) == ORC_INVALID_ARGUMENT
    assert oracle.check_row(12, 256, 144) == 0


def test_live_reference_random_rows():
    """Fresh seeded rows through the compiled reference, bit for bit (when it is built)."""
    if not oracle.ref_available():
        pytest.skip("compiled reference not built")
    rng = np.random.default_rng(99)
    rows, cols = 16, 2048
    x = rng.standard_normal(cols).astype(np.float32)
    for t in (13, 14, 8):
        data = synth.weights(t, rng, rows, cols)
        y_ref = oracle.ref_storage_matvec(t, rows, cols, data, x)
        y_orc = oracle.storage_matvec(t, rows, cols, data, x)
        y_mt = oracle.storage_matvec(t, rows, cols, data, x, threads=4)
        assert np.array_equal(y_ref.view(np.uint32), y_orc.view(np.uint32))
        assert np.array_equal(y_ref.view(np.uint32), y_mt.view(np.uint32))
        for r in range(0, rows, 5):
            row = data.reshape(rows, -1)[r]
            assert np.array_equal(oracle.ref_decode_row(t, cols, row).view(np.uint32),
                                  oracle.decode_row(t, cols, row).view(np.uint32))
    q5 = synth.q5_k(rng, rows, cols).reshape(-1, 176)
    q5[:, 16:48] = 0
    q4 = np.concatenate([q5[:, :16], q5[:, 48:]], axis=1).reshape(-1)
    y5 = oracle.ref_storage_matvec(13, rows, cols, q5.reshape(-1), x)
    y4 = oracle.storage_matvec(12, rows, cols, q4, x)
    assert np.array_equal(y5.view(np.uint32), y4.view(np.uint32))


# ---------------------------------------------------------------- tolerance normaliser, helpers

def _plain_rows(t, rng, rows, cols):
    """Seeded rows of an unquantized type (f32 = 0, f16 = 1, bf16 = 30) as raw bytes."""
    v = rng.standard_normal((rows, cols)).astype(np.float32) * 0.05
    if t == 0:
        return v.view(np.uint8).reshape(-1)
    if t == 1:
        return v.astype(np.float16).view(np.uint8).reshape(-1)
    return (v.view(np.uint32) >> 16).astype("<u2").view(np.uint8).reshape(-1)


def _normaliser_agrees(got_dot, got_abs, want_dot, want_abs):
    """The stats agree with a float64 recomputation to 1e-12 of the row's sum |w x|."""
    scale = np.maximum(want_abs, 1e-300)
    return bool(np.all(np.abs(got_abs - want_abs) <= 1e-12 * scale)
                and np.all(np.abs(got_dot - want_dot) <= 1e-12 * scale))


@pytest.mark.parametrize("t", [0, 1, 30, 8, 12, 13, 14])
def test_matvec_stats_is_float64_sum_over_decoded_rows(t):
    """orc_storage_matvec_stats / orc_storage_dot_stats (the per-output bar of every product test)
    equal numpy's float64 sum of w*x and of |w*x| over the rows decode_row gives (decode_row is
    pinned to the compiled reference above), at ragged sizes; wrong normalisers are rejected."""
    rng = np.random.default_rng(4100 + t)
    block = {0: 1, 1: 1, 30: 1, 8: 32}.get(t, 256)
    for rows, cols in ((1, block * 3), (7, 2 * 1024 + block), (33, 4096)):
        if t in (0, 1, 30):
            data = _plain_rows(t, rng, rows, cols + 5)
            cols = cols + 5
        else:
            data = synth.weights(t, rng, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        x[rng.integers(0, cols, 3)] = 0.0
        w = oracle.decode_matrix(t, cols, rows, data).astype(np.float64)
        prod = w * x.astype(np.float64)[None, :]
        want_dot, want_abs = prod.sum(axis=1), np.abs(prod).sum(axis=1)
        for threads in (1, 3):
            dot, ab = oracle.matvec_stats(t, rows, cols, data, x, threads=threads)
            assert _normaliser_agrees(dot, ab, want_dot, want_abs), (t, rows, cols, threads)
        rb = data.size // rows
        for r in (0, rows - 1):
            d1, a1 = C_stats_dot(t, cols, data[r * rb:(r + 1) * rb], x)
            assert _normaliser_agrees(np.array([d1]), np.array([a1]), want_dot[r:r + 1], want_abs[r:r + 1])
        # planted mistakes the check must reject: sum|w| * max|x|, |sum w x|, sum of |w| * |x| over
        # only the first half of the row
        wrong = [np.abs(w).sum(axis=1) * np.abs(x).max(), np.abs(want_dot),
                 np.abs(prod[:, : cols // 2]).sum(axis=1)]
        for bad in wrong:
            assert not _normaliser_agrees(want_dot, bad, want_dot, want_abs), t


def C_stats_dot(t, n, row, x):
    import ctypes as C
    d = np.ascontiguousarray(row, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    dot, ab = C.c_double(), C.c_double()
    rc = oracle.lib().orc_storage_dot_stats(t, n, d.ctypes.data, d.nbytes, xv.ctypes.data, C.byref(dot), C.byref(ab))
    assert rc == 0
    return dot.value, ab.value


def test_matvec_stats_errors_follow_matvec():
    x = np.ones(256, np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.matvec_stats(13, 2, 256, np.zeros(351, np.uint8), x)
    with pytest.raises(oracle.OracleError):
        oracle.matvec_stats(13, 0, 256, np.zeros(352, np.uint8), x)


def test_fnv1a64_published_vectors():
    """FNV-1a 64-bit: offset basis 0xcbf29ce484222325, prime 0x100000001b3 (the published
    test vectors of the FNV reference page)."""
    assert oracle.fnv1a64(b"") == 0xCBF29CE484222325
    assert oracle.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64(b"foobar") == 0x85944171F73967E8
    # and against a direct restatement on random bytes
    blob = np.random.default_rng(7).integers(0, 256, 1000, dtype=np.uint8).tobytes()
    h = 0xCBF29CE484222325
    for b in blob:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    assert oracle.fnv1a64(blob) == h


@pytest.mark.parametrize("t", [8, 12, 13, 14])
def test_storage_matmul_is_m_matvecs(t):
    """orc_storage_matmul_mt with m > 1 is m independent reference matvecs
    (src/runtime/qwen35_target_multi.cpp:14-25): row i of the output equals, bit for bit, the
    matvec of activation row i (itself bit-equal to the compiled reference), for any thread count."""
    rng = np.random.default_rng(4200 + t)
    rows, cols, m = 11, 1024 if t != 8 else 96, 5
    data = synth.weights(t, rng, rows, cols)
    x = rng.standard_normal((m, cols)).astype(np.float32)
    for threads in (1, 4):
        y = oracle.storage_matmul(t, rows, cols, data, x, threads=threads)
        assert y.shape == (m, rows)
        for i in range(m):
            want = oracle.storage_matvec(t, rows, cols, data, x[i])
            assert np.array_equal(y[i].view(np.uint32), want.view(np.uint32)), (t, threads, i)
            if oracle.ref_available() and t != 12:
                ref = oracle.ref_storage_matvec(t, rows, cols, data, x[i])
                assert np.array_equal(y[i].view(np.uint32), ref.view(np.uint32))
    # a transposed activation (columns and rows swapped) gives a different product: the check sees it
    yt = oracle.storage_matmul(t, rows, cols, data, np.ascontiguousarray(x[::-1]))
    assert not np.array_equal(yt[0], y[0])
