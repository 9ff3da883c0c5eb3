"""Oracle formats (encoders / unpack) pinned by the reference's own tests and
closed forms; the library's host encoders must agree bit for bit."""
import numpy as np
import pytest

from rapidocrvl_amd import lib

Q8, Q4, Q6 = 1000, 1001, 1002


def test_round_to_int_ties(orc):
    # internal/tensor/quant_test.go:107-118
    for x, want in [(1.49, 1), (1.50, 2), (-1.49, -1), (-1.50, -2), (0.0, 0)]:
        assert orc.round_to_int(x) == want


def test_value_tables(orc):
    # q4Value / q4ByteLo / q4ByteHi / q8Value / q6Value (quant_test.go:119-128)
    every = np.arange(256, dtype=np.uint8)
    lo_hi = orc.unpack_matrix(Q4, every.reshape(256, 1), 2)
    assert (lo_hi[:, 0] == (every & 15).astype(np.int16) - 8).all()
    assert (lo_hi[:, 1] == (every >> 4).astype(np.int16) - 8).all()
    assert lo_hi[0xF0, 0] == -8 and lo_hi[0xF0, 1] == 7 and lo_hi[0x08, 0] == 0
    q8 = orc.unpack_row(Q8, every, 256)
    assert q8[0x80] == -128 and q8[0] == 0 and q8[127] == 127
    assert (q8 == every.view(np.int8)).all()
    # one 6-bit code per row: codes 0, 32, 63 → -32, 0, 31
    for code, want in [(0, -32), (32, 0), (63, 31)]:
        assert orc.unpack_row(Q6, np.array([code], np.uint8), 1)[0] == want


def test_q6_unpack_exhaustive(orc):
    # every 3-byte group (2^24) decodes to its four little-endian 6-bit fields − 32
    v = np.arange(1 << 24, dtype=np.uint32)
    row = np.stack([v & 255, (v >> 8) & 255, (v >> 16) & 255], axis=1).astype(np.uint8).reshape(-1)
    got = orc.unpack_row(Q6, row, 4 << 24).reshape(-1, 4).astype(np.int32)
    for k in range(4):
        assert (got[:, k] == ((v >> (6 * k)) & 63).astype(np.int32) - 32).all()


def test_q6_pack_round_trip_odd_cols(orc):
    # quant_test.go:87-98: code (i*7)&63 at col i survives pack/unpack for 11 cols
    cols = 11
    codes = np.array([(i * 7) & 63 for i in range(cols)], np.int32)
    # w chosen so that round(w*inv) = code-32 exactly: inv = 1 when maxAbs = 31
    w = (codes - 32).astype(np.float32)
    w[0] = -31.0 if abs(w).max() < 31 else w[0]
    scale, row = orc.quantize_row(Q6, w)
    assert scale == np.float32(abs(w).max() / np.float32(31))
    assert (orc.unpack_row(Q6, row, cols) == np.clip(np.round(w / scale), -31, 31)).all()


def test_q4_odd_cols_tail_nibble_cleared(orc):
    # quant_test.go:61-67
    _, row = orc.quantize_row(Q4, np.array([1, -1, 0.5], np.float32))
    assert row.size == 2 and row[1] & 0xF0 == 0


def test_q8_bytes_known_answer(orc):
    # quant_test.go:26-41 inputs; scale 3/127, codes round-half-away(w*127/3)
    w = np.array([1, -2, 3, 0.5, 0.25, -0.75, 0], np.float32)
    scale, row = orc.quantize_row(Q8, w)
    assert scale == np.float32(3) / np.float32(127)
    assert list(row.view(np.int8)) == [42, -85, 127, 21, 11, -32, 0]


def test_q4_known_answer(orc):
    w = np.array([1, -2, 3, 0.5, 0.25, -0.75, 0], np.float32)
    scale, row = orc.quantize_row(Q4, w)
    assert scale == np.float32(3) / np.float32(7)
    # nibbles 10,3 | 15,9 | 9,6 | 8 (codes 2,-5,7,1,1,-2,0)
    assert list(row) == [10 | 3 << 4, 15 | 9 << 4, 9 | 6 << 4, 8]


@pytest.mark.parametrize("qtype,lim", [(Q4, 7), (Q6, 31)])
def test_tie_modes(orc, qtype, lim):
    # maxAbs = lim → scale 1, inv 1: w*inv is exactly the half-integer
    w = np.array([lim, 0.5, 2.5, -0.5, -2.5, 1.5, 0, 0], np.float32)
    away = orc.unpack_row(qtype, orc.quantize_row(qtype, w, orc.TIE_HALF_AWAY)[1], 8)
    even = orc.unpack_row(qtype, orc.quantize_row(qtype, w, orc.TIE_AMD64)[1], 8)
    assert list(away) == [lim, 1, 3, -1, -3, 2, 0, 0]
    assert list(even) == [lim, 0, 2, 0, -2, 2, 0, 0]


def test_q8_tie_mode_is_half_away_always(orc):
    w = np.array([127, 0.5, 2.5, -0.5, -2.5, 1.5, 0, 0], np.float32)
    for tie in (orc.TIE_HALF_AWAY, orc.TIE_AMD64):
        assert list(orc.quantize_row(Q8, w, tie)[1].view(np.int8)) == [127, 1, 3, -1, -3, 2, 0, 0]


@pytest.mark.parametrize("qtype,zero", [(Q8, 0), (Q4, -8), (Q6, -32)])
def test_all_zero_row(orc, qtype, zero):
    scale, row = orc.quantize_row(qtype, np.zeros(9, np.float32))
    assert scale == 1.0 and not row.any()
    assert (orc.unpack_row(qtype, row, 9) == zero).all()


def test_codes_bounded_and_reconstruct(orc, rng):
    # |code·scale − w| ≤ scale/2 (+f32 slack) and |code| ≤ qmax: the defining property
    for qtype, qmax in [(Q8, 127), (Q4, 7), (Q6, 31)]:
        w = (rng.standard_normal((64, 77)) * 0.02).astype(np.float32)
        sc, data = orc.quantize_matrix(qtype, w)
        codes = orc.unpack_matrix(qtype, data, 77).astype(np.float64)
        assert np.abs(codes).max() <= qmax
        err = np.abs(codes * sc[:, None].astype(np.float64) - w)
        assert (err <= sc[:, None] * (0.5 + 1e-5)).all()
        assert np.allclose(np.abs(w).max(axis=1) / qmax, sc, rtol=1e-7)


@pytest.mark.parametrize("cols", [1, 2, 3, 5, 8, 11, 16, 31, 64, 100, 1024, 3072])
@pytest.mark.parametrize("qtype", [Q8, Q4, Q6])
@pytest.mark.parametrize("tie", [0, 1])
def test_library_encoder_matches_oracle(orc, rng, cols, qtype, tie):
    w = (rng.standard_normal((9, cols)) * 0.02).astype(np.float32)
    w[3] = 0  # all-zero row
    if cols > 2:
        w[4, :2] = [0.5, -0.5]  # exact ties once scaled
        w[4, 2] = 7.0
    s_lib, p_lib = lib.quantize_rows(qtype, w, tie)
    s_orc, p_orc = orc.quantize_matrix(qtype, w, tie)
    assert s_lib.tobytes() == s_orc.tobytes()
    assert p_lib.tobytes() == p_orc.tobytes()
    assert (lib.unpack_rows(qtype, p_lib, cols) == orc.unpack_matrix(qtype, p_orc, cols)).all()


def test_row_bytes(orc):
    for cols in range(1, 40):
        assert orc.row_bytes(Q8, cols) == lib.row_bytes(Q8, cols) == cols
        assert orc.row_bytes(Q4, cols) == lib.row_bytes(Q4, cols) == (cols + 1) // 2
        assert orc.row_bytes(Q6, cols) == lib.row_bytes(Q6, cols) == (6 * cols + 7) // 8
