"""Pins the CPU oracle (oracle/oracle.py) before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle (a dropped term,
a wrong sign or index, a wrong rounding/summation order) fails one of them:
golden vectors from the independent scalar C oracle, hand-derived known
answers, closed forms and brute force on tiny inputs.
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import oracle as O

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
DIMS = (32, 64, 128, 256)


# ---------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("d", DIMS)
def test_encode_matches_golden(d):
    x = GOLDEN[f"enc_d{d}_x"]
    b = O.binary_encode(x)
    assert np.array_equal(b.words, GOLDEN[f"enc_d{d}_words"])
    assert np.array_equal(b.scale.view(np.uint16), GOLDEN[f"enc_d{d}_scale"])
    r = O.residual_encode(x, b)
    assert np.array_equal(r.codes, GOLDEN[f"enc_d{d}_codes"])
    assert np.array_equal(r.scale.view(np.uint16), GOLDEN[f"enc_d{d}_rscale"])
    _, ro = O.online_encode(x)
    assert np.array_equal(ro.codes, GOLDEN[f"enc_d{d}_codes_online"])
    assert np.array_equal(ro.scale.view(np.uint16), GOLDEN[f"enc_d{d}_rscale_online"])


@pytest.mark.parametrize("d", DIMS)
def test_scores_match_golden(d):
    q = GOLDEN[f"qs_d{d}_q"]
    k = GOLDEN[f"qs_d{d}_k"]
    qw, sq, _ = O.query_prep(q)
    assert np.array_equal(qw, GOLDEN[f"qs_d{d}_qwords"])
    assert np.array_equal(sq.view(np.uint32), GOLDEN[f"qs_d{d}_scale_q"].view(np.uint32))
    _, sqt, _ = O.query_prep_tree(q)
    assert np.array_equal(sqt.view(np.uint32), GOLDEN[f"qs_d{d}_scale_q_tree"].view(np.uint32))
    kb = O.binary_encode(k)
    for i in range(q.shape[0]):
        pc = O.popcounts(qw[i], kb.words)
        assert np.array_equal(pc, GOLDEN[f"qs_d{d}_pc"][i])
        xd = O.xnor_dot(sq[i], pc, kb.scale, d)
        assert np.array_equal(xd.view(np.uint32), GOLDEN[f"qs_d{d}_xdot"][i].view(np.uint32))
    ent = O.head_entropy(q[:, None, :].reshape(1, 3, d), O.BinaryEnc(
        np.tile(kb.words, (3, 1)), np.tile(kb.scale, 3), np.tile(kb.mean32, 3)), 1, 3, 40)
    np.testing.assert_allclose(ent[0], GOLDEN[f"qs_d{d}_entropy"], rtol=2e-6, atol=2e-6)


# ---------------------------------------------------------------- known answers
def test_sign_kats():
    x = np.full((1, 32), 1.0, np.float16)
    assert O.binary_encode(x).words[0, 0] == 0xFFFFFFFF
    alt = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float16)[None]
    assert list(O.binary_encode(alt).words[0]) == [0x55555555, 0x55555555]
    z = np.array([[0.0, -0.0] * 16], np.float16)
    b = O.binary_encode(z)
    assert b.words[0, 0] == 0xFFFFFFFF and float(b.scale[0]) == 0.0
    nan = np.full((1, 32), np.nan, np.float16)
    assert O.binary_encode(nan).words[0, 0] == 0


def test_scale_closed_form():
    # constant |x| = c: the mean is exactly c (sums of equal powers of two)
    for d in DIMS:
        for c in (0.5, 0.125, 3.0, 2.0 ** -10):
            x = np.full((1, d), c, np.float16)
            x[0, ::3] *= -1
            assert float(O.binary_encode(x).scale[0]) == c


def test_scale_tree_order_differs_from_sequential():
    # choose values where the 128-thread tree order and a sequential sum round
    # differently; the oracle must follow the tree (agreement with the C oracle
    # which simulates the block literally).
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4000, 128)) * 100).astype(np.float16)
    b = O.binary_encode(x)
    seq = np.zeros(4000, np.float32)
    for i in range(128):
        seq = (seq + np.abs(x[:, i].astype(np.float32))).astype(np.float32)
    differs = (seq / np.float32(128)) != b.mean32
    assert differs.any()          # the order is observable
    w, s, m = C.binary_encode(x)
    assert np.array_equal(m.view(np.uint32), b.mean32.view(np.uint32))


# ---------------------------------------------------------------- fp32 order KATs
# Hand-derived known answers for the three fp32 operation orders that fix the
# encoded bytes and the binary scores.  Each input is chosen so that the
# reference's order and the plausible alternatives round to different fp32
# bits; the expected bits are worked out by hand in the comments (ulp(1) =
# 2^-23 in fp32, 2^-10 in fp16; ties round to even).

def _bits(v) -> int:
    return int(np.asarray(v, np.float32).view(np.uint32))


def _f32_round(x: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to fp32 (normal range)."""
    if x == 0:
        return np.float32(0.0)
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (e - 23)
    n, rem = divmod(a, ulp)
    n = int(n)
    if rem / ulp > Fraction(1, 2) or (rem / ulp == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(float((1 if x > 0 else -1) * n * ulp))


def test_encode_scale_tree_order_kat():
    """src/binary_encode.cu:31-53: 128 threads, p_t = |x_t| (+ |x_{t+128}|),
    then p_t += p_{t+s} for s = 64 .. 1.

    d = 128, x = [1, 2^-11, 2^-24 x 126].  Tree: s=64 gives p0 = 1 + 2^-24 ->
    1 (tie, even), p1 = 2^-11 + 2^-24, p2..63 = 2^-23; each later level adds
    a doubled power of two to p0 and p1 exactly, so before s=1 p0 = 1 +
    31*2^-23 and p1 = 2^-11 + 63*2^-24; s=1 gives 1 + 2^-11 + 62.5*2^-23 ->
    1 + 2^-11 + 62*2^-23 (tie, even mantissa 4158).  mean = that / 128 =
    0x3C00103E; fp16 of it lies above the midpoint 2^-7*(1 + 2^-11), so the
    scale is 2^-7*(1 + 2^-10) = 0x2001.
    A left-to-right sum keeps 1 + 2^-11 (each + 2^-24 is a tie to even),
    mean 2^-7*(1 + 2^-11), fp16 tie -> 0x2000.  An exact sum gives
    1 + 2^-11 + 63*2^-23 (mean 0x3C00103F).
    d = 64, x = [1, 2^-11, 2^-24 x 62]: p0 = 1 + 15*2^-23, p1 = 2^-11 +
    31*2^-24 before s=1, total 1 + 2^-11 + 30*2^-23 (tie at 30.5, even),
    mean 0x3C80101E, scale 2^-6*(1 + 2^-10) = 0x2401 (left to right: 0x2400)."""
    for d, mean_bits, scale_bits, seq_scale in ((128, 0x3C00103E, 0x2001, 0x2000),
                                                (64, 0x3C80101E, 0x2401, 0x2400)):
        row = [1.0, 2.0 ** -11] + [2.0 ** -24] * (d - 2)
        for sign in (1.0, -1.0):                # |x|: the signs must not matter
            x = (np.array([row], np.float32) * sign).astype(np.float16)
            b = O.binary_encode(x)
            assert _bits(b.mean32[0]) == mean_bits, (d, hex(_bits(b.mean32[0])))
            assert int(b.scale.view(np.uint16)[0]) == scale_bits
            _, _, m = C.binary_encode(x)
            assert _bits(m[0]) == mean_bits
        # the alternatives named above round differently
        seq = np.float32(0.0)
        for v in row:
            seq = np.float32(seq + np.float32(v))
        assert int(np.float16(seq / np.float32(d)).view(np.uint16)) == seq_scale != scale_bits
        exact = _f32_round(sum(Fraction(v) for v in row) / d)
        assert _bits(exact) != mean_bits


def test_scale_q_sequential_order_kat():
    """src/compensated_attention.cu:65-67 (and binary_attention.cu:34-36):
    scale_q = (sequential fp32 sum of |q_i|) / d; src/adaptive_precision.cu:46-59
    (entropy) uses the encode's tree order instead.

    d = 128, q = [1, 2^-24 x 127].  Left to right every + 2^-24 is a tie that
    rounds back to 1, so scale_q = 2^-7 = 0x3C000000.  Tree order (as in the
    encode KAT): 1 + (1+2+4+8+16+32)*2^-23 = 1 + 63*2^-23, scale 0x3C00003F.
    Right to left: 127*2^-24 exactly, then + 1 -> 1 + 63.5*2^-23 -> 1 +
    64*2^-23 (tie, even), 0x3C000040.
    With a key of all-positive signs and scale 1 (popcount 128) the binary
    score is (2^-7 * 1) * 128 * inv_sqrt_d = inv_sqrt_d exactly."""
    q = np.array([[1.0] + [2.0 ** -24] * 127], np.float16)
    _, sq, _ = O.query_prep(q)
    _, sqt, _ = O.query_prep_tree(q)
    assert _bits(sq[0]) == 0x3C000000
    assert _bits(sqt[0]) == 0x3C00003F
    rev = np.float32(0.0)
    for v in q[0, ::-1].astype(np.float32):
        rev = np.float32(rev + v)
    assert _bits(rev / np.float32(128)) == 0x3C000040
    _, csq = C.query_prep(q)
    _, csqt = C.query_prep(q, tree=True)
    assert _bits(csq[0]) == 0x3C000000 and _bits(csqt[0]) == 0x3C00003F
    k = np.ones((1, 128), np.float16)
    s = O.binary_scores(q.reshape(1, 1, 128), O.binary_encode(k), 1, 1, 1)
    assert _bits(s[0, 0, 0]) == _bits(O.inv_sqrt(128)) == 0x3DB504F3


def test_xnor_score_association_kat():
    """src/xnor_dot.cuh:28-30: xdot = (scale_q * scale_k) * (float)(2pc - d).

    scale_q = 1 + 3*2^-23, scale_k = 1 + 2^-10 (fp16), 2pc - d = 6.
    (scale_q*scale_k) = 1 + 2^-10 + 3*2^-23 (+ 3*2^-33, dropped); times 6 =
    6 + 6*2^-10 + 18*2^-23: at exponent 2 the ulp is 2^-21, so the tail is
    4.5 ulps -> 4 (tie, even): 6 + 6*2^-10 + 2^-19 = 0x40C03004.
    scale_q * (scale_k*6) rounds only once, from 4.5 ulps + 18*2^-33 (above
    the tie) -> 5 ulps: 0x40C03005.
    End to end: q = [127, 1, 3*2^-16, 0 x 125] gives the sequential sum
    128 + 3*2^-16 (exact) and scale_q = 0x3F800003; the key [+c x 67,
    -c x 61] with c = 1 + 2^-10 has scale c (0x3C01) and popcount 67, so
    the score is fp32(0x40C03004 * inv_sqrt(128)) = 0x3F07E5AA."""
    sq = np.float32(1 + 3 * 2.0 ** -23)
    sk = np.array([1 + 2.0 ** -10], np.float16)
    xd = O.xnor_dot(sq, np.array([67], np.int32), sk, 128)
    assert _bits(xd[0]) == 0x40C03004
    other = np.float32(sq * np.float32(np.float32(sk[0]) * np.float32(6)))
    assert _bits(other) == 0x40C03005
    fr = Fraction(float(sq)) * Fraction(float(sk[0]))
    assert _bits(_f32_round(Fraction(float(_f32_round(fr))) * 6)) == 0x40C03004
    q = np.array([[127.0, 1.0, 3 * 2.0 ** -16] + [0.0] * 125], np.float16)
    _, sqq, _ = O.query_prep(q)
    assert _bits(sqq[0]) == 0x3F800003
    c = 1 + 2.0 ** -10
    kb = O.binary_encode(np.array([[c] * 67 + [-c] * 61], np.float16))
    assert int(kb.scale.view(np.uint16)[0]) == 0x3C01
    s = O.binary_scores(q.reshape(1, 1, 128), kb, 1, 1, 1)
    assert _bits(s[0, 0, 0]) == 0x3F07E5AA
    assert _bits(_f32_round(Fraction(float(xd[0])) * Fraction(float(O.inv_sqrt(128))))) == 0x3F07E5AA
    qw, csq = C.query_prep(q)
    pc, cxd = C.xnor_scores(qw[0], float(csq[0]), kb.words, kb.scale, 128)
    assert pc[0] == 67 and _bits(cxd[0]) == 0x40C03004


def test_residual_kats():
    # x = s + e with s the fp16 mean: residual codes at exact half-steps round half to even.
    d = 32
    # bits all 1, mean = 1.0 ; residuals r_i = x_i - 1
    r = np.zeros(d, np.float32)
    r[0] = 0.5       # absmax
    r[1] = -0.5
    r[2] = 0.5 / 14  # r*7/absmax = 0.5  -> 0 (half to even)
    r[3] = 1.5 / 14  # 1.5 -> 2
    r[4] = 2.5 / 14  # 2.5 -> 2
    r[5:] = 0.0
    # build x so that the mean stays 1.0: add compensating values pairwise
    x = (1.0 + r).astype(np.float32)
    x[6], x[7] = 1.0 - r[2], 1.0 - r[3]
    x[8] = 1.0 - r[4]
    x16 = x.astype(np.float16)[None]
    b = O.binary_encode(x16)
    s = float(b.scale[0])
    rr = x16.astype(np.float32)[0] - s
    enc = O.residual_encode(x16, b)
    absmax = np.max(np.abs(rr))
    exp = np.clip(np.rint(rr * np.float32(7.0 / absmax)), -7, 7)
    assert np.array_equal(enc.codes[0], exp.astype(np.int8))
    # absmax = 0 -> all codes 0 and scale 0
    const = np.full((1, 64), 0.75, np.float16)
    e = O.residual_encode(const, O.binary_encode(const))
    assert (e.codes == 0).all() and float(e.scale[0]) == 0.0
    # the element at absmax always maps to +-7
    rng = np.random.default_rng(1)
    x = rng.standard_normal((200, 128)).astype(np.float16)
    b = O.binary_encode(x)
    e = O.residual_encode(x, b)
    assert (np.abs(e.codes).max(axis=1) == 7).all()


def test_residual_reconstruction_bound():
    rng = np.random.default_rng(2)
    for d in DIMS:
        x = (rng.standard_normal((300, d)) * 0.3).astype(np.float16)
        b = O.binary_encode(x)
        e = O.residual_encode(x, b)
        rec = O.dequant_binary(b, d) + O.dequant_residual(e)
        err = np.abs(rec - x.astype(np.float32))
        # half a quantisation step plus the fp16 rounding of absmax (<= 2^-11 relative)
        bound = e.scale.astype(np.float32)[:, None] * (1 / 14 + 2.0 ** -11) * 1.0001 + 1e-7
        assert (err <= bound).all()


def test_online_vs_two_step_differ_only_through_scale():
    # B4: the online path uses the fp32 mean; when the mean is exactly
    # representable in fp16 both paths are identical.
    x = np.full((1, 128), 0.5, np.float16)
    x[0, 5] = -0.5
    b, r_on = O.online_encode(x)
    r_two = O.residual_encode(x, b)
    assert np.array_equal(r_on.codes, r_two.codes)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5000, 128)).astype(np.float16)
    b, r_on = O.online_encode(x)
    r_two = O.residual_encode(x, b)
    diff = (r_on.codes != r_two.codes).any(axis=1)
    exact = b.mean32 == b.scale.astype(np.float32)
    assert not diff[exact].any()
    assert diff.any()


def test_nibble_pack_roundtrip_and_layout():
    codes = np.arange(-7, 8, dtype=np.int8)
    codes = np.concatenate([codes, codes[:1]])[None]          # 16 values
    nib = O.pack_nibbles(codes)
    assert nib[0, 0] == ((-7 & 0xF) | ((-6 & 0xF) << 4))
    assert np.array_equal(O.unpack_nibbles(nib), codes)


# ---------------------------------------------------------------- scores
@pytest.mark.parametrize("d", DIMS)
def test_popcount_closed_form(d):
    rng = np.random.default_rng(d)
    q = rng.standard_normal((4, d)).astype(np.float16)
    k = rng.standard_normal((50, d)).astype(np.float16)
    qw, sq, q32 = O.query_prep(q)
    kb = O.binary_encode(k)
    sgn_q = np.where(q.astype(np.float32) >= 0, 1, -1)
    sgn_k = np.where(k.astype(np.float32) >= 0, 1, -1)
    dots = sgn_q @ sgn_k.T
    for i in range(4):
        pc = O.popcounts(qw[i], kb.words)
        assert np.array_equal(2 * pc - d, dots[i])
    # q == k -> d ; q == -k -> -d
    pc = O.popcounts(qw[0], O.binary_encode(q[:1]).words)
    assert pc[0] == d
    neg = (-q[:1].astype(np.float32)).astype(np.float16)
    neg[neg == 0] = np.float16(-1.0)  # avoid +-0 which both map to bit 1
    qq = q[:1].copy()
    qq[qq == 0] = np.float16(1.0)
    qwq, _, _ = O.query_prep(qq)
    assert O.popcounts(qwq[0], O.binary_encode(neg).words)[0] == 0


def test_scale_q_sequential_closed_form():
    # powers of two with <= 24 significant bits in total: every partial sum is exact
    q = np.array([[2.0 ** -i if i < 20 else 0.0 for i in range(32)]], np.float16)
    _, sq, _ = O.query_prep(q)
    exact = sum(2.0 ** -i for i in range(20))
    assert float(sq[0]) == exact / 32


def test_compensated_scores_closed_form():
    """score = [(sq*sgn q).(sk*sgn k) + q.(n/7*rs)] / sqrt(d), evaluated in float64
    by matmul over decoded K, must match the oracle's per-key restatement."""
    rng = np.random.default_rng(7)
    B, H, S, d = 1, 2, 64, 128
    Q = (rng.standard_normal((B, H, d)) * 0.1).astype(np.float16)
    K = (rng.standard_normal((B * H * S, d)) * 0.1).astype(np.float16)
    V = (rng.standard_normal((B * H * S, d)) * 0.1).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    out, o32 = O.compensated_attention(Q, Kb, Kr, Vb, Vr, B, H, S, return_f32=True)
    qw, sq, q32 = O.query_prep(Q.reshape(-1, d))
    Kbin = O.dequant_binary(Kb, d).astype(np.float64).reshape(B * H, S, d)
    Kres = O.dequant_residual(Kr).astype(np.float64).reshape(B * H, S, d)
    Vrec = (O.dequant_binary(Vb, d) + O.dequant_residual(Vr)).astype(np.float64).reshape(B * H, S, d)
    for i in range(B * H):
        qb = sq[i] * np.where(q32[i] >= 0, 1.0, -1.0)
        s = (Kbin[i] @ qb + Kres[i] @ q32[i].astype(np.float64)) / math.sqrt(d)
        w = np.exp(s - s.max())
        ref = (w @ Vrec[i]) / w.sum()
        np.testing.assert_allclose(o32.reshape(B * H, d)[i], ref, rtol=1e-4, atol=1e-6)
    # exact-order literal restatement agrees with the vectorised one
    for i in range(B * H):
        sl = slice(i * S, (i + 1) * S)
        ex = O.compensated_attention_exact_order(
            Q.reshape(-1, d)[i], O.BinaryEnc(Kb.words[sl], Kb.scale[sl], Kb.mean32[sl]),
            O.ResidualEnc(Kr.codes[sl], Kr.scale[sl]), O.BinaryEnc(Vb.words[sl], Vb.scale[sl], Vb.mean32[sl]),
            O.ResidualEnc(Vr.codes[sl], Vr.scale[sl]), S)
        np.testing.assert_allclose(o32.reshape(B * H, d)[i], ex, rtol=2e-5, atol=2e-7)


def test_binary_attention_closed_form():
    """Binary attention over random keys in float64 from the decoded signs:
    score = sq * sk * (sgn q . sgn k) / sqrt(d) with sq = mean|q| and sk the
    fp16 scale, out = softmax-weighted (+-sv).  Pins the score scale (a
    dropped scale_q, scale_k or 1/sqrt(d), or a wrong sign convention, moves
    the weights) and the binary V reconstruction."""
    rng = np.random.default_rng(17)
    for d, S in ((64, 200), (128, 300), (256, 150)):
        B, H = 1, 3
        Q = (rng.standard_normal((B, H, d)) * 3.0).astype(np.float16)
        K = (rng.standard_normal((B * H * S, d)) * 1.5 *
             np.exp(rng.standard_normal((B * H * S, 1)) * 0.5)).astype(np.float16)
        V = (rng.standard_normal((B * H * S, d)) * 0.5).astype(np.float16)
        Kb = O.binary_encode(K)
        Vb = O.binary_encode(V)
        _, o32 = O.binary_attention(Q, Kb, Vb, B, H, S, return_f32=True)
        sk = Kb.scale.astype(np.float64).reshape(B * H, S)
        sv = Vb.scale.astype(np.float64).reshape(B * H, S)
        sgk = np.where(K.astype(np.float64) >= 0, 1.0, -1.0).reshape(B * H, S, d)
        sgv = np.where(V.astype(np.float64) >= 0, 1.0, -1.0).reshape(B * H, S, d)
        for i in range(B * H):
            q = Q.reshape(-1, d)[i].astype(np.float64)
            sq = np.abs(q).mean()
            s = sq * sk[i] * (sgk[i] @ np.where(q >= 0, 1.0, -1.0)) / math.sqrt(d)
            w = np.exp(s - s.max())
            ref = (w @ (sv[i][:, None] * sgv[i])) / w.sum()
            np.testing.assert_allclose(o32.reshape(B * H, d)[i], ref, rtol=2e-5, atol=1e-6)
        # the scores span many nats, so the test is not blind to their scale
        assert np.ptp(s) > 4.0


def test_torch_cpu_restatement_matches_oracle():
    """compensated_attention_torch_cpu (the CPU baseline's and the full-size
    c3 test's fast path) against the numpy oracle on the same encodings."""
    import torch
    rng = np.random.default_rng(19)
    d, S = 128, 700
    Q = (rng.standard_normal((1, 1, d)) * 0.2).astype(np.float16)
    K = (rng.standard_normal((S, d)) * 0.2).astype(np.float16)
    V = (rng.standard_normal((S, d)) * 0.2).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    _, ref = O.compensated_attention(Q, Kb, Kr, Vb, Vr, 1, 1, S, return_f32=True)
    w64 = lambda w: torch.from_numpy(w.astype(np.int64))
    got = O.compensated_attention_torch_cpu(
        torch.from_numpy(Q[0, 0]), w64(Kb.words), torch.from_numpy(Kb.scale),
        torch.from_numpy(Kr.codes.astype(np.int8)), torch.from_numpy(Kr.scale),
        w64(Vb.words), torch.from_numpy(Vb.scale), torch.from_numpy(Vr.codes.astype(np.int8)),
        torch.from_numpy(Vr.scale))
    np.testing.assert_allclose(got.float().numpy(), ref[0, 0].astype(np.float16).astype(np.float32),
                               rtol=2e-3, atol=2e-4)


def test_torch_cpu_binary_and_adaptive_restatements_match_oracle():
    """binary_attention_torch_cpu and adaptive_attention_torch_cpu (the fast
    paths of the full-size c2 and c5 GPU checks) against the numpy oracle on
    the same encodings: GQA rows sharing a kv head, repeated key rows so that
    the top-k threshold falls inside tie groups, and a NaN / -0 / +inf K
    scale for the selection's ordering rules.  Sets must be equal; outputs
    agree to fp16 rounding."""
    import torch
    rng = np.random.default_rng(31)
    d, S, G = 128, 700, 4
    Q = (rng.standard_normal((1, G, d)) * 0.2).astype(np.float16)
    base = (rng.standard_normal((S // 3, d)) * 0.2).astype(np.float16)
    K = base[rng.integers(0, base.shape[0], S)]
    V = (rng.standard_normal((S, d)) * 0.2).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    w64 = lambda w: torch.from_numpy(w.astype(np.int64))
    t = torch.from_numpy
    args_k = (w64(Kb.words), t(Kb.scale))
    args_v = (w64(Vb.words), t(Vb.scale))
    _, ref = O.binary_attention(Q, Kb, Vb, 1, G, S, n_kv_heads=1, return_f32=True)
    got = O.binary_attention_torch_cpu(t(Q[0]), *args_k, *args_v)
    np.testing.assert_allclose(got.float().numpy(), ref[0].astype(np.float16).astype(np.float32),
                               rtol=2e-3, atol=2e-4)
    for top_k in (1, 70, 233, S - 1):
        _, ref, sets = O.adaptive_attention(Q, Kb, Kr, Vb, Vr, 1, G, S, top_k, n_kv_heads=1,
                                            return_f32=True, return_sets=True)
        got, sel = O.adaptive_attention_torch_cpu(
            t(Q[0]), *args_k, t(Kr.codes.astype(np.int8)), t(Kr.scale), *args_v,
            t(Vr.codes.astype(np.int8)), t(Vr.scale), top_k)
        for h in range(G):
            assert np.array_equal(np.flatnonzero(sel[h].numpy()), sets[(0, h)]), (top_k, h)
        np.testing.assert_allclose(got.float().numpy(), ref[0].astype(np.float16).astype(np.float32),
                                   rtol=2e-3, atol=2e-4)
    # special scales: the selection's ordering only (outputs are not finite)
    ks = Kb.scale.copy()
    ks[[3, 10, 11, 50]] = np.array([np.nan, -0.0, np.inf, 0.0], np.float16)
    Kb2 = O.BinaryEnc(Kb.words, ks, ks.astype(np.float32))
    with np.errstate(all="ignore"):
        _, _, sets = O.adaptive_attention(Q, Kb2, Kr, Vb, Vr, 1, G, S, 90, n_kv_heads=1,
                                          return_f32=True, return_sets=True)
        _, sel = O.adaptive_attention_torch_cpu(
            t(Q[0]), w64(Kb2.words), t(ks), t(Kr.codes.astype(np.int8)), t(Kr.scale), *args_v,
            t(Vr.codes.astype(np.int8)), t(Vr.scale), 90)
    for h in range(G):
        assert np.array_equal(np.flatnonzero(sel[h].numpy()), sets[(0, h)]), h


def test_attention_special_cases():
    rng = np.random.default_rng(9)
    d = 64
    # S = 1 -> output is the V reconstruction
    Q = rng.standard_normal((1, 1, d)).astype(np.float16)
    K = rng.standard_normal((1, d)).astype(np.float16)
    V = rng.standard_normal((1, d)).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    out, o32 = O.compensated_attention(Q, Kb, Kr, Vb, Vr, 1, 1, 1, return_f32=True)
    vrec = O.dequant_binary(Vb, d) + O.dequant_residual(Vr)
    np.testing.assert_allclose(o32[0, 0], vrec[0], rtol=1e-6)
    # all keys identical -> equal weights -> mean of V reconstructions
    S = 37
    K = np.repeat(K, S, axis=0)
    V = rng.standard_normal((S, d)).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    _, o32 = O.compensated_attention(Q, Kb, Kr, Vb, Vr, 1, 1, S, return_f32=True)
    vrec = O.dequant_binary(Vb, d) + O.dequant_residual(Vr)
    np.testing.assert_allclose(o32[0, 0], vrec.mean(axis=0), rtol=1e-5, atol=1e-7)
    _, b32 = O.binary_attention(Q, Kb, Vb, 1, 1, S, return_f32=True)
    np.testing.assert_allclose(b32[0, 0], O.dequant_binary(Vb, d).mean(axis=0), rtol=1e-5, atol=1e-7)


def test_gqa_equals_mha_on_repeated_kv():
    rng = np.random.default_rng(11)
    B, Hq, Hkv, S, d = 2, 4, 2, 33, 64
    Q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    K = rng.standard_normal((B, Hkv, S, d)).astype(np.float16)
    V = rng.standard_normal((B, Hkv, S, d)).astype(np.float16)
    Kb, Kr = O.encode_fused(K.reshape(-1, d))
    Vb, Vr = O.encode_fused(V.reshape(-1, d))
    gqa = O.compensated_attention(Q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv)
    Kx = np.repeat(K, Hq // Hkv, axis=1).reshape(-1, d)
    Vx = np.repeat(V, Hq // Hkv, axis=1).reshape(-1, d)
    Kb2, Kr2 = O.encode_fused(Kx)
    Vb2, Vr2 = O.encode_fused(Vx)
    mha = O.compensated_attention(Q, Kb2, Kr2, Vb2, Vr2, B, Hq, S)
    assert np.array_equal(gqa.view(np.uint16), mha.view(np.uint16))


def test_entropy_closed_form():
    rng = np.random.default_rng(13)
    B, H, S, d = 1, 3, 500, 128
    Q = rng.standard_normal((B, H, d)).astype(np.float16)
    K = rng.standard_normal((B * H * S, d)).astype(np.float16)
    Kb = O.binary_encode(K)
    ent = O.head_entropy(Q, Kb, B, H, S)
    qw, sq, _ = O.query_prep_tree(Q.reshape(-1, d))
    for h in range(H):
        sl = slice(h * S, (h + 1) * S)
        pc = O.popcounts(qw[h], Kb.words[sl])
        s = (sq[h] * Kb.scale[sl].astype(np.float64)) * (2 * pc - d)
        p = np.exp(s - s.max())
        p /= p.sum()
        H_ref = -(p * np.log(np.where(p > 0, p, 1))).sum()
        assert abs(ent[0, h] - H_ref) < 1e-4 * max(1.0, abs(H_ref))


def test_reference_attention_closed_form():
    rng = np.random.default_rng(17)
    B, H, S, d = 1, 2, 70, 64
    Q = rng.standard_normal((B, H, d)).astype(np.float16)
    K = rng.standard_normal((B, H, S, d)).astype(np.float16)
    V = rng.standard_normal((B, H, S, d)).astype(np.float16)
    _, o32 = O.reference_attention(Q, K, V, B, H, S, return_f32=True)
    for h in range(H):
        s = K[0, h].astype(np.float64) @ Q[0, h].astype(np.float64) / math.sqrt(d)
        w = np.exp(s - s.max())
        ref = w @ V[0, h].astype(np.float64) / w.sum()
        np.testing.assert_allclose(o32[0, h], ref, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- top-k
def test_topk_bruteforce_and_ties():
    key = np.array([3, 1, 3, 2, 3, 0, -1, 3], np.float32)
    assert list(O.topk_select(key, 3)) == [0, 2, 4]
    assert list(O.topk_select(key, 5)) == [0, 2, 3, 4, 7]
    rng = np.random.default_rng(19)
    for _ in range(50):
        S = int(rng.integers(1, 60))
        key = rng.integers(-3, 4, S).astype(np.float32) * np.float32(0.5)
        k = int(rng.integers(0, S + 1))
        sel = O.topk_select(key, k)
        # brute force: rank = number of keys strictly better (greater, or equal with lower index)
        ranks = [sum(1 for j in range(S) if key[j] > key[i] or (key[j] == key[i] and j < i)) for i in range(S)]
        assert set(sel) == {i for i in range(S) if ranks[i] < k}


def test_topk_key_canonicalisation_and_exactness():
    ks = np.array([0.0, 1.5, np.nan, 65504.0], np.float16)
    pc = np.array([10, 64, 64, 0], np.int32)
    key = O.topk_key(ks, pc, 128)
    assert np.signbit(key[0]) == False  # -0 -> +0
    assert key[2] == -np.inf
    assert key[3] == np.float32(65504.0) * np.float32(-128)
    assert O.default_top_k(131072) == 13108
    assert O.default_top_k(30) == 3 and O.default_top_k(31) == 4


def test_adaptive_all_selected_equals_compensated_and_none_equals_binary():
    rng = np.random.default_rng(23)
    B, Hq, Hkv, S, d = 1, 4, 2, 50, 128
    Q = (rng.standard_normal((B, Hq, d)) * 0.3).astype(np.float16)
    K = (rng.standard_normal((B * Hkv * S, d)) * 0.3).astype(np.float16)
    V = (rng.standard_normal((B * Hkv * S, d)) * 0.3).astype(np.float16)
    Kb, Kr = O.encode_fused(K)
    Vb, Vr = O.encode_fused(V)
    _, a32 = O.adaptive_attention(Q, Kb, Kr, Vb, Vr, B, Hq, S, S, n_kv_heads=Hkv, return_f32=True)
    _, c32 = O.compensated_attention(Q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    np.testing.assert_allclose(a32, c32, rtol=1e-6, atol=1e-7)
    _, a0 = O.adaptive_attention(Q, Kb, Kr, Vb, Vr, B, Hq, S, 0, n_kv_heads=Hkv, return_f32=True)
    _, b0 = O.binary_attention(Q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    np.testing.assert_allclose(a0, b0, rtol=1e-6, atol=1e-7)


def test_adaptive_attention_closed_form_between_the_limits():
    """O.adaptive_attention at 0 < k < S, MHA and GQA, with ties at the
    threshold, against a float64 closed form built from the raw inputs: the
    selected set by a lexsort on scale_k * (sgn q . sgn k) (largest first,
    lowest index on ties), the score sq*sk*(sgn q . sgn k)/sqrt(d) plus, for
    selected keys only, q . deq(K_res)/sqrt(d), and V = +-sv plus, for
    selected keys only, deq(V_res).  A slip that pairs residual rows with the
    wrong keys (first k rows, a transposed index, another head's set) moves
    the output.  Intent: src/adaptive_precision.cuh:6-12; score
    src/xnor_dot.cuh:30."""
    rng = np.random.default_rng(29)
    d = 128
    for B, Hq, Hkv, S in ((1, 3, 3, 300), (2, 4, 2, 260)):
        n = B * Hkv * S
        # few distinct rows repeated in random order: many keys tie exactly
        base = (rng.standard_normal((n // 4, d)) * 0.3).astype(np.float16)
        K = base[rng.integers(0, base.shape[0], n)]
        V = (rng.standard_normal((n, d)) * 0.3).astype(np.float16)
        Q = (rng.standard_normal((B, Hq, d)) * 0.3).astype(np.float16)
        Kb, Kr = O.encode_fused(K)
        Vb, Vr = O.encode_fused(V)
        sgn = lambda a: np.where(a.astype(np.float64) >= 0, 1.0, -1.0)
        sk = Kb.scale.astype(np.float64).reshape(B, Hkv, S)
        kres = (Kr.codes.astype(np.float64) / 7 * Kr.scale.astype(np.float64)[:, None]).reshape(B, Hkv, S, d)
        vres = (Vr.codes.astype(np.float64) / 7 * Vr.scale.astype(np.float64)[:, None]).reshape(B, Hkv, S, d)
        vbin = (sgn(V) * Vb.scale.astype(np.float64)[:, None]).reshape(B, Hkv, S, d)
        ksg = sgn(K).reshape(B, Hkv, S, d)
        g = Hq // Hkv
        keys = {}
        for b in range(B):
            for h in range(Hq):
                keys[(b, h)] = sk[b, h // g] * (ksg[b, h // g] @ sgn(Q[b, h]))
        # a k whose threshold falls inside a tie group of the first head
        order0 = np.lexsort((np.arange(S), -keys[(0, 0)]))
        kv = keys[(0, 0)][order0]
        top_k = next(k for k in range(S // 10, S - 1) if kv[k - 1] == kv[k])
        straddles = 0
        out, o32, sets = O.adaptive_attention(Q, Kb, Kr, Vb, Vr, B, Hq, S, top_k, n_kv_heads=Hkv,
                                              return_f32=True, return_sets=True)
        for b in range(B):
            for h in range(Hq):
                key = keys[(b, h)]
                order = np.lexsort((np.arange(S), -key))
                sel = np.zeros(S, bool)
                sel[order[:top_k]] = True
                straddles += key[order[top_k - 1]] == key[order[top_k]]
                assert np.array_equal(np.flatnonzero(sel), sets[(b, h)]), (b, h)
                assert not np.array_equal(np.flatnonzero(sel), np.arange(top_k))
                q = Q[b, h].astype(np.float64)
                sq = np.abs(q).mean()
                sc = (sq * key + sel * (kres[b, h // g] @ q)) / math.sqrt(d)
                vrec = vbin[b, h // g] + sel[:, None] * vres[b, h // g]
                w = np.exp(sc - sc.max())
                ref = (w @ vrec) / w.sum()
                np.testing.assert_allclose(o32[b, h], ref, rtol=1e-4, atol=2e-6 * np.abs(ref).max())
                # the residual terms matter at this k: the binary-only and
                # fully compensated outputs differ from the adaptive one
                scb = sq * key / math.sqrt(d)
                wb = np.exp(scb - scb.max())
                assert np.abs((wb @ vbin[b, h // g]) / wb.sum() - ref).max() > 50 * 1e-4 * np.abs(ref).max()
        assert straddles >= 1


def test_ring_state():
    r = O.RingState(3)
    slots = [r.append() for _ in range(7)]
    assert slots == [0, 1, 2, 0, 1, 2, 0]
    assert r.filled == 3 and r.write_pos == 1


def test_kendall_tau_ab_against_brute_force():
    """The O(n log n) tau-a / tau-b helper against the reference's O(n^2)
    pair loop (tests/test_correctness.cu:58-71) on tied and untied data."""
    from bitcache_amd.workloads import kendall_tau_ab
    rng = np.random.default_rng(23)
    for x, y in ((rng.standard_normal(300), rng.standard_normal(300)),
                 (rng.integers(0, 5, 200).astype(float), rng.integers(0, 7, 200).astype(float))):
        y = y + 0.5 * x
        c = dsc = 0
        for i in range(len(x)):
            for j in range(i + 1, len(x)):
                p = (x[i] - x[j]) * (y[i] - y[j])
                c += p > 0
                dsc += p < 0
        n0 = len(x) * (len(x) - 1) / 2
        n1 = sum(t * (t - 1) / 2 for t in np.unique(x, return_counts=True)[1])
        n2 = sum(t * (t - 1) / 2 for t in np.unique(y, return_counts=True)[1])
        ta, tb = kendall_tau_ab(x, y)
        assert abs(ta - (c - dsc) / n0) < 1e-9
        assert abs(tb - (c - dsc) / math.sqrt((n0 - n1) * (n0 - n2))) < 1e-9
