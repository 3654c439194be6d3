"""Known-answer blocks for the weight quantizers BlockQ4K::from_float
(fuel-quantized/src/k_quants.rs:1470-1528, make_qkx1_quants utils.rs:229-286)
and BlockQ6K::from_float (k_quants.rs:2005-2075, make_qx_quants utils.rs:62-226
with rmse_type 1), worked out by hand.  Test helper only.

Each block is built so that the search provably lands on a value fixed by the
mathematics, not by re-running the algorithm:

* Q4K, "grid" sub-blocks: x = (l - a) * s with s a power of two, integer a >= 0
  and codes l in [0, 15] with both 0 and 15 present.  Then min = -a*s,
  max - min = 15*s, iscale = 15 / (15*s) = 1/s exactly, every first-pass code is
  l, sum(x - min)*l / sum(l*l) = s exactly (all partial sums are small integers
  times s), the mean residual is exactly -a*s, and the second pass changes
  nothing: make_qkx1_quants returns (s, a*s) exactly.
* Q6K, "grid" groups: x = q * s with s a power of two, q in [-32, 31] and
  q = -32 at exactly one element (the unique max |x|).  Then iscale =
  -32 / (-32*s) = 1/s, the first codes are q, sum(w x l) / sum(w l l) = s exactly
  (w = x*x; every term is q^4 times a power of two and the partial sums stay
  below 2^24), the refinement loop sees no change, and the coordinate-descent
  proposal x*sl2/slx equals q up to two roundings: make_qx_quants returns s.
  A group whose max |x| is positive (q in [-31, 32], +32 present) gives
  iscale = -1/s, codes -q and scale -s by the same argument.

Everything after the search (the 6-bit / int8 scale quantization, the f16
d / dmin and the final codes) is then arithmetic on those exact values; the
expected bytes below carry the hand results, and `code_margin` confirms that
no final code sits near a rounding boundary, so the expectations are not
fragile.  The plausible slips each block catches are listed with it.
"""
from __future__ import annotations

import numpy as np

import oracle as O


def round_half_away(v: float) -> int:
    """Rust f32::round (utils.rs:1-3 nearest_int), on an exactly known value."""
    return int(np.sign(v) * np.floor(abs(v) + 0.5))


def f16_bits(v32: np.float32) -> int:
    """half::f16::from_f32 of an f32 value: IEEE round-to-nearest-even (numpy's
    float32 -> float16 conversion, itself pinned against F16C in
    test_oracle_rng_f16)."""
    return int(np.float32(v32).astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# Q4K
# ---------------------------------------------------------------------------

def _pack_q4k_scales(ls, lm):
    """GGUF 6-bit packing of 8 (scale, min) pairs: the inverse of
    get_scale_min_k4 (utils.rs:50-60), whose decoding test_oracle_quant pins
    on crafted blocks."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= ls[j]
            s[j + 4] |= lm[j]
        else:
            s[j + 4] |= (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    return s


def _pack_q4k_codes(codes):
    q = [0] * 128
    for c in range(4):
        for i in range(32):
            q[32 * c + i] = codes[64 * c + i] | (codes[64 * c + 32 + i] << 4)
    return q


def _q4k_block(d_bits, dmin_bits, ls, lm, codes):
    b = np.zeros(1, O.BLOCK_Q4K)
    b["d"] = d_bits
    b["dmin"] = dmin_bits
    b["scales"] = np.array(_pack_q4k_scales(ls, lm), np.uint8)
    b["qs"] = np.array(_pack_q4k_codes(codes), np.uint8)
    return b


# codes 0..15 twice, in an order that differs per sub-block
def _grid_codes(j):
    base = np.concatenate([np.arange(16), np.arange(15, -1, -1)])
    return np.roll(base, 5 * j).astype(np.int64)


Q4K_S = 2.0 ** -6  # the block's largest sub-block scale


def q4k_grid_case():
    """Eight grid sub-blocks (s_j, a_j):

      j  s      a    make_qkx1   ls = round(63 s/S)   lm = round(63 a s / 63S)
      0  S      0    (S, 0)      63                   0
      1  S      7    (S, 7S)     63                   7
      2  S/2    2    (S/2, S)    round(31.5) = 32     1
      3  S      63   (S, 63S)    63                   63    <- max min
      4  S/4    4    (S/4, S)    round(15.75) = 16    1
      5  S/128  0    (S/128, 0)  round(0.49) = 0      0     <- codes stay 0
      6  S/2    21   (S/2,10.5S) 32                   round(10.5) = 11 (half away)
      7  S      30   (S, 30S)    63                   30

    d = f16(S/63), dmin = f16(63S/63) = f16(S).  Codes: l, except sub-block 5
    (ls = 0: d = 0, the codes keep their initial 0) and sub-block 6, where the
    min's rounding up by half a step (11 S against 10.5 S, one code step of
    S/2) shifts every code up by one: l + 1, clamped at 15.

    Catches: a wrong grid min or max (sign of the min, min/max swapped), an
    inexact iscale, ls/lm rounding to even (sub-block 6 gives lm 10), the
    6-bit packing order, d / dmin swapped, codes not clamped at 15, codes of a
    zero-scale sub-block written.
    """
    S = Q4K_S
    sj = [S, S, S / 2, S, S / 4, S / 128, S / 2, S]
    aj = [0, 7, 2, 63, 4, 0, 21, 30]
    x = np.zeros(256, np.float32)
    want_codes = np.zeros(256, np.int64)
    lcodes = []
    for j in range(8):
        l = _grid_codes(j)
        lcodes.append(l)
        x[32 * j:32 * j + 32] = ((l - aj[j]) * sj[j]).astype(np.float32)
    ls = [63, 63, 32, 63, 16, 0, 32, 63]
    lm = [0, 7, 1, 63, 1, 0, 11, 30]
    for j in range(8):
        c = lcodes[j]
        if j == 5:
            c = np.zeros(32, np.int64)
        elif j == 6:
            c = np.minimum(c + 1, 15)
        want_codes[32 * j:32 * j + 32] = c
    d_bits = f16_bits(np.float32(S) / np.float32(63))
    dmin_bits = f16_bits(np.float32(63 * S) / np.float32(63))
    assert dmin_bits == f16_bits(np.float32(S))
    return x, _q4k_block(d_bits, dmin_bits, ls, lm, want_codes)


def q4k_edge_case():
    """Edge sub-blocks:

      j  data                                make_qkx1          ls   lm
      0  32 x 0.375 (constant)               max == min: (0,0)  0    0
      1  +0.0 / -0.0 alternating             max == min: (0,0)  0    0
         (total_cmp orders -0 < +0 but f32 == holds; comparing the bit
         patterns instead would reach 15/0 and NaN scales, which the scale
         quantization also maps to 0: the bytes do not tell them apart)
      2  l*S, l in 1..15 (all positive)      min clamped to 0   63   0
                                             before the search:
                                             (S, -0.0)
      3  (l + 1/8)*S/2, l in 0..15           min clamped to 0   32   0
                                             at the start and after the
                                             first pass (mean residual
                                             +0.0171 S): (0.50605 S, -0.0)
      4  (l - 1)*S                           (S, S)             63   63  <- max min
      5  l*S/4                               (S/4, 0)           16   0
      6  (l - 1)*S/4                         (S/4, S/4)         16   16
      7  all -0.5 (constant, negative)       (0, 0)             0    0

    d = f16(S/63), dmin = f16(S/63).  Codes: 0 for sub-blocks 0, 1, 7 (ls = 0);
    l for 2, 4, 5, 6; l for 3 as well ((l + 1/8) * 63/64 rounds to l).

    Catches: either `min > 0 -> 0` clamp dropped (sub-block 2 then searches from min = S
    and its lm turns negative; sub-block 3's lm becomes -1 -> byte 255), a
    constant sub-block encoded with its value.
    """
    S = Q4K_S
    x = np.zeros(256, np.float32)
    x[0:32] = 0.375
    x[32:64] = np.where(np.arange(32) % 2 == 0, np.float32(0.0), np.float32(-0.0))
    l_pos = np.roll(np.concatenate([np.arange(1, 16), np.arange(15, 0, -1), [7, 9]]), 3).astype(np.int64)
    x[64:96] = (l_pos * S).astype(np.float32)
    l3 = _grid_codes(3)
    x[96:128] = ((l3 + 0.125) * (S / 2)).astype(np.float32)
    l4 = _grid_codes(4)
    x[128:160] = ((l4 - 1) * S).astype(np.float32)
    l5 = _grid_codes(5)
    x[160:192] = (l5 * (S / 4)).astype(np.float32)
    l6 = _grid_codes(6)
    x[192:224] = ((l6 - 1) * (S / 4)).astype(np.float32)
    x[224:256] = -0.5
    ls = [0, 0, 63, 32, 63, 16, 16, 0]
    lm = [0, 0, 0, 0, 63, 0, 16, 0]
    codes = np.zeros(256, np.int64)
    codes[64:96] = l_pos
    codes[96:128] = l3
    codes[128:160] = l4
    codes[160:192] = l5
    codes[192:224] = l6
    d_bits = f16_bits(np.float32(S) / np.float32(63))
    return x, _q4k_block(d_bits, d_bits, ls, lm, codes)


def q4k_zero_case():
    """All-zero superblock: every sub-block is constant -> (0, 0); d = dmin =
    f16(0 / 63) = +0; all 144 bytes zero."""
    return np.zeros(256, np.float32), np.zeros(1, O.BLOCK_Q4K)


# ---------------------------------------------------------------------------
# Q6K
# ---------------------------------------------------------------------------

def _pack_q6k(d_bits, scales, codes):
    """codes: stored values L = q + 32 in [0, 63] (k_quants.rs:2043-2062)."""
    b = np.zeros(1, O.BLOCK_Q6K)
    ql = np.zeros(128, np.int64)
    qh = np.zeros(64, np.int64)
    for h in range(2):
        L = codes[128 * h:128 * h + 128]
        for i in range(32):
            ql[64 * h + i] = (L[i] & 0xF) | ((L[i + 64] & 0xF) << 4)
            ql[64 * h + 32 + i] = (L[i + 32] & 0xF) | ((L[i + 96] & 0xF) << 4)
            qh[32 * h + i] = (L[i] >> 4) | ((L[i + 32] >> 4) << 2) | ((L[i + 64] >> 4) << 4) | \
                ((L[i + 96] >> 4) << 6)
    b["ql"] = ql.astype(np.uint8)
    b["qh"] = qh.astype(np.uint8)
    b["scales"] = np.array(scales, np.int8)
    b["d"] = d_bits
    return b


def _q6_grid(g, rng):
    """16 codes in [-31, 31] with one -32 (the unique max |x|) at a position
    that moves with g."""
    q = rng.integers(-31, 32, 16)
    q[(5 * g + 3) % 16] = -32
    return q.astype(np.int64)


Q6K_S = 2.0 ** -5


def q6k_grid_case():
    """Sixteen groups (s_g):  make_qx_quants returns s_g; the first group with
    the largest |s| is group 0 (s = S), so iscale = -128/S, d = f16(-S/128) =
    -2^-12 exactly (bits 0x8C00) and scale byte g = round(-128 s_g / S) clamped
    at 127:

      g   s        scale byte           codes (stored L)
      0   S        -128                 q + 32
      1   -S       round(128) -> 127    q + 32 (128q/127 rounds to q)
      2   S/2      -64                  q + 32
      3   -S/4     32                   q + 32
      4   S/1024   round(-0.125) = 0    q + 32 from the search (d = 0: kept)
      5   zeros    0                    0 (the all-zero branch writes 0)
      6   S/8      -16                  q + 32
      7   -S/2     64                   q + 32
      8   S, max |x| positive:          scale -S -> byte 127, codes -q + 32
          q in [-31, 32] with +32       (x / d = 128 q / 127 * -1 rounds to -q)
      9   S/4      -32                  q + 32
      10  -S       127                  q + 32
      11  S/16     -8                   q + 32
      12  S/2      -64                  q + 32
      13  -S/8     16                   q + 32
      14  S        -128                 q + 32
      15  S/32     -4                   q + 32

    Catches: the sign convention of iscale (-nmax / max with the signed max),
    the first-strictly-greater choice of the max |scale| (group 1 ties group
    0's |s|; taking it would flip d's sign), the 127 saturation, codes of a
    group whose scale byte rounds to 0 (kept from the search, not 32), the
    zero group writing 0 rather than 32, the ql / qh interleave.
    """
    S = Q6K_S
    rng = np.random.default_rng(20240614)
    sg = [S, -S, S / 2, -S / 4, S / 1024, 0.0, S / 8, -S / 2, S, S / 4, -S, S / 16, S / 2, -S / 8, S, S / 32]
    x = np.zeros(256, np.float32)
    codes = np.zeros(256, np.int64)
    scales = [0] * 16
    for g in range(16):
        q = _q6_grid(g, rng)
        if g == 5:
            x[16 * g:16 * g + 16] = 0.0
            codes[16 * g:16 * g + 16] = 0
            scales[g] = 0
            continue
        if g == 8:
            q = -q  # q in [-31, 32], +32 present: the max |x| is positive
            x[16 * g:16 * g + 16] = (q * sg[g]).astype(np.float32)
            codes[16 * g:16 * g + 16] = -q + 32
            scales[g] = 127
            continue
        x[16 * g:16 * g + 16] = (q * sg[g]).astype(np.float32)
        codes[16 * g:16 * g + 16] = q + 32
        scales[g] = min(round_half_away(-128.0 * sg[g] / S), 127)
    assert scales[:5] == [-128, 127, -64, 32, 0]
    return x, _pack_q6k(0x8C00, scales, codes)


def q6k_tie_case():
    """Group 0 has s = -S and group 1 s = +S (equal |s|): the first one is
    max_scale = -S, so iscale = 128/S and d = f16(S/128) = +2^-12 (0x0C00);
    bytes: group 0 -128, group 1 round(128) -> 127.  Others S/2 (byte 64)."""
    S = Q6K_S
    rng = np.random.default_rng(7)
    x = np.zeros(256, np.float32)
    codes = np.zeros(256, np.int64)
    scales = []
    for g in range(16):
        s = -S if g == 0 else S if g == 1 else S / 2
        q = _q6_grid(g, rng)
        x[16 * g:16 * g + 16] = (q * s).astype(np.float32)
        codes[16 * g:16 * g + 16] = q + 32
        scales.append(-128 if g == 0 else 127 if g == 1 else round_half_away(128.0 * s / S))
    assert scales[2] == 64
    return x, _pack_q6k(0x0C00, scales, codes)


def q6k_zero_case():
    """All-zero superblock: every group scale is 0, so max_scale = 0,
    iscale = -128/0 = -inf, d = f16(1/-inf) = -0.0 (bits 0x8000), scale bytes
    round(-inf * 0 = NaN) as i32 = 0, codes 0."""
    b = np.zeros(1, O.BLOCK_Q6K)
    b["d"] = 0x8000
    return np.zeros(256, np.float32), b


# ---------------------------------------------------------------------------
# Q4K from_float_imatrix: the importance formula
# ---------------------------------------------------------------------------

IMX_QB = 3.0  # importance of the zero elements of sub-blocks 4..7


def q4k_imatrix_formula_case():
    """A block whose bytes depend on the importance formula of
    BlockQ4K::from_float_imatrix (k_quants.rs:1539-1548):

      sigma2 = 2 * sum(x^2) / 256,   w_l = imatrix_l * sqrt(sigma2 + x_l^2),
      sw_j = sum over sub-block j of w_l.

    Sub-blocks 0..3 ("A"): x = -15 at element 0, 0 elsewhere (a grid with step
    1 from min -15, codes 0 and 15): make_qkx3_quants (utils.rs:358-469) fits
    it with zero error at its first pass, so it returns (1, 15) for any
    weights.  Sub-blocks 4..7 ("B"): x = -1, 14, then 30 zeros (grid from min
    -1, codes 0, 15, 1): (1, 1).  sum(x^2) = 4*225 + 4*197 = 1688, sigma2 =
    13.1875 exactly.

    Importance: 1 on each A sub-block's -15 (x^2 = 225 >> sigma2), IMX_QB on
    each B sub-block's 30 zeros (x^2 = 0 << sigma2), 1e-3 elsewhere.  So sw_A
    follows |x| and barely sigma2, sw_B follows sqrt(sigma2): the factor 2 and
    the square root set the ratio sw_B / sw_A.

    make_qp_quants (utils.rs:472-563) over the eight scales (all 1) gives codes
    63 and d = 1/63 -> f16 bits 9232.  Over the mins (15 x 4, 1 x 4): max 15,
    iscale 63/15 = 4.2, codes 63 and round(4.2) = 4 for every candidate
    iscale of the search ((63 + 0.1 is) and (4.2 + is/150) round to 63 and 4
    for |is| <= 4), and the coordinate descent keeps them (its proposals
    m_j * sl2 / slx stay inside (62.5, 63.5] and (3.5, 4.5): `imatrix_margins`).
    The result is the weighted least-squares fit

      dmin = (945 W_A + 4 W_B) / (3969 W_A + 16 W_B),  W_A = sum_{j<4} sw_j,
                                                      W_B = sum_{j>=4} sw_j,

    evaluated in float64 and rounded to f16 (its distance from the f16
    rounding boundary is checked by `imatrix_margins`).  Codes: A -> 0 at the
    -15 and 15 elsewhere, B -> 0, 15, then 1 ((x + dmin*m) / (d*sc) with d*sc
    ~ 1 and dmin*m ~ 15.06 / 0.956).

    With sigma2 = sum(x^2)/256 the same closed form gives dmin bits 2 below,
    without the square root 6 below: either slip changes the bytes.
    """
    x, qw = imatrix_formula_inputs()
    dmin = imatrix_formula_dmin(x, qw)
    ls = [63] * 8
    lm = [63, 63, 63, 63, 4, 4, 4, 4]
    codes = np.full(256, 15, np.int64)
    for j in range(4):
        codes[32 * j] = 0
    for j in range(4, 8):
        codes[32 * j:32 * j + 32] = 1
        codes[32 * j] = 0
        codes[32 * j + 1] = 15
    d_bits = f16_bits(np.float32(1.0) / np.float32(63))
    return x, qw, _q4k_block(d_bits, int(np.float16(dmin).view(np.uint16)), ls, lm, codes)


def imatrix_formula_inputs():
    x = np.zeros(256, np.float32)
    qw = np.full(256, 1e-3, np.float32)
    for j in range(4):
        x[32 * j] = -15.0
        qw[32 * j] = 1.0
    for j in range(4, 8):
        x[32 * j] = -1.0
        x[32 * j + 1] = 14.0
        qw[32 * j + 2:32 * j + 32] = IMX_QB
    return x, qw


def imatrix_formula_sw(x, qw, sigma2_factor=2.0, sqrt=True):
    """sw_j of the block in float64; the keyword arguments give the slips."""
    x = x.astype(np.float64)
    sigma2 = sigma2_factor * float(np.sum(x * x)) / 256.0
    t = sigma2 + x * x
    return (qw.astype(np.float64) * (np.sqrt(t) if sqrt else t)).reshape(8, 32).sum(1)


IMX_MINS = np.array([15, 15, 15, 15, 1, 1, 1, 1], np.float64)
IMX_LM = np.array([63, 63, 63, 63, 4, 4, 4, 4], np.float64)


def imatrix_formula_dmin(x, qw, **slip):
    sw = imatrix_formula_sw(x, qw, **slip)
    wa, wb = sw[:4].sum(), sw[4:].sum()
    return (945.0 * wa + 4.0 * wb) / (3969.0 * wa + 16.0 * wb)


def imatrix_margins(x, qw):
    """(f16 margin of dmin in ulps, worst descent-proposal margin): the first
    is the distance of the float64 dmin from the nearest f16 rounding boundary
    (0.5 = on an f16 value), the second the smallest distance of a proposal
    m_j * sl2 / slx (the fit without element j, utils.rs:540-553) from the
    boundary that would change its code."""
    dmin = imatrix_formula_dmin(x, qw)
    ulp = 2.0 ** (np.floor(np.log2(dmin)) - 10)
    u = dmin / ulp
    f16_margin = abs((u - np.floor(u)) - 0.5)
    sw = imatrix_formula_sw(x, qw)
    worst = 1.0
    for j in range(8):
        keep = np.arange(8) != j
        slx = float((sw * IMX_MINS * IMX_LM)[keep].sum())
        sl2 = float((sw * IMX_LM * IMX_LM)[keep].sum())
        p = IMX_MINS[j] * sl2 / slx
        if j < 4:
            worst = min(worst, p - 62.5)  # anything above rounds to 63 or is clamped to it
        else:
            worst = min(worst, p - 3.5, 4.5 - p)
    return f16_margin, worst


CASES = {
    "q4k_grid": (O.Q4K, q4k_grid_case),
    "q4k_edge": (O.Q4K, q4k_edge_case),
    "q4k_zero": (O.Q4K, q4k_zero_case),
    "q6k_grid": (O.Q6K, q6k_grid_case),
    "q6k_tie": (O.Q6K, q6k_tie_case),
    "q6k_zero": (O.Q6K, q6k_zero_case),
}


def code_margin(dt: int, x: np.ndarray, block: np.ndarray) -> float:
    """Largest distance of an unclamped final code's real value
    (x + dmin*m) / (d*sc) from its rounded integer, in float64 from the
    expected block's own fields: the hand results above stay clear of the
    rounding boundaries when this is well below 0.5."""
    from blockref import q4k_fields, q6k_fields

    worst = 0.0
    if dt == O.Q4K:
        d, dmin, sc, mn, q = q4k_fields(block)
        for j in range(8):
            dj = float(np.float32(d[0]) * np.float32(sc[0, j]))
            if dj == 0.0:
                continue
            dm = float(np.float32(dmin[0]) * np.float32(mn[0, j]))
            t = (x[32 * j:32 * j + 32].astype(np.float64) + dm) / dj
            r = np.clip(t, 0, 15)
            worst = max(worst, float(np.abs(r - np.round(r)).max()))
    else:
        d, sc, q = q6k_fields(block)
        for g in range(16):
            dj = float(np.float32(d[0]) * np.float32(sc[0, g]))
            if dj == 0.0:
                continue
            t = x[16 * g:16 * g + 16].astype(np.float64) / dj
            r = np.clip(t, -32, 31)
            worst = max(worst, float(np.abs(r - np.round(r)).max()))
    return worst
