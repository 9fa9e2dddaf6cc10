"""Hand-derived float32 vectors that pin the oracle's elementwise functions
bit for bit: fastExp, GELUQuick, Softmax, RMSNorm and the RoPE rotation.

Each function below is float32 arithmetic in the reference's Go source, one
rounding per operation (Go on amd64 with the default GOAMD64=v1 does not fuse
a*b+c).  The GPU kernels are tested bit-exact against the oracle, so these
vectors are what fixes the GPU's elementwise results to the reference's
statements:

- fastExp (internal/kernels/activation.go:100-145): clamp at +-10, y = x*log2e,
  i = int32(y) (truncation toward zero, :115), f = y - float32(i), the Horner
  polynomial with four float32 coefficients (:121-126), times 2^i built from
  exponent bits (:134-137).
- GELUQuickSIMD (activation.go:47-95): sx = 1.702*x; sigmoid = 1/(1+fastExp(-sx))
  when sx >= 0 (:64-67), else e/(1+e) with e = fastExp(sx) (:68-72); x*sigmoid.
- Softmax (activation.go:161-213): e_i = fastExp(x_i - max); per group of four
  `sum += e0 + e1 + e2 + e3` (:192), i.e. sum + (((e0+e1)+e2)+e3); the tail is
  added one by one; then dst *= 1/sum (:209-212).
- RMSNorm (internal/kernels/norm.go:8-36): sumSq = eight FMA lanes and the hsum
  ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) (simd_amd64.s:19-76); meanSq = sumSq /
  float32(n); rms = float32(math.Sqrt(float64(meanSq+eps))); invRms = 1/rms;
  dst = VecScaleF32 then VecMulF32, i.e. (x*invRms)*w with two roundings.
- RoPE (internal/kernels/rope_cache.go:102-103): x0' = v0*cos - v1*sin and
  x1' = v0*sin + v1*cos, each product rounded before the add.

How the expected values were derived.  Every value is a float32, written as an
integer multiple of a power of two.  An operation's exact result is a rational
number; it is rounded to nearest (ties to even) at the binade's ulp, and the
docstring of each pin walks the steps.  The constants are the Go untyped
constants converted to float32 (correctly rounded, as the Go spec requires):

  log2e  1.442695041         -> 0x3FB8AA3B = 12102203 * 2^-23
  c1     0.693147180559945   -> 0x3F317218 = 11629080 * 2^-24
  c2     0.240226506959101   -> 0x3E75FDF0 = 16121328 * 2^-26
  c3     0.055504108664821   -> 0x3D635847 = 14899271 * 2^-28
  c4     0.009676036358193   -> 0x3C1E883D = 10389565 * 2^-30
  1.702                      -> 0x3FD9DB23
  eps    1e-6 (GGUF default)  -> 0x358637BD

`model_*` below is an exact-rational model of the same statements with knobs;
the tests use it to re-derive every expected value and to show that each
plausible mistake (a knob turned) changes at least one pinned value.  The pins
themselves are the hex constants in PINS.
"""
from __future__ import annotations

import dataclasses
import math
import struct
from fractions import Fraction

F = Fraction


# ------------------------------------------------------- exact rounding ----

def rnd(q, p: int = 24, emin: int = -126) -> Fraction:
    """Round a rational to p significant bits, nearest-even (IEEE binary32
    for p = 24, emin = -126; binary64 for 53, -1022)."""
    q = F(q)
    if q == 0:
        return F(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if F(2) ** e > a:
        e -= 1
    elif F(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = F(2) ** (e - (p - 1))
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > F(1, 2) or (rem == F(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


def r32(q) -> Fraction:
    return rnd(q, 24, -126)


def r64(q) -> Fraction:
    return rnd(q, 53, -1022)


def sqrt_rnd(q, p: int) -> Fraction:
    """sqrt(q) for a positive rational q, correctly rounded to p bits."""
    q = F(q)
    e = (q.numerator.bit_length() - q.denominator.bit_length()) // 2
    while F(2) ** (2 * e) > q:
        e -= 1
    while F(2) ** (2 * (e + 1)) <= q:
        e += 1
    ulp = F(2) ** (e - (p - 1))
    t = q / (ulp * ulp)
    n = math.isqrt(t.numerator // t.denominator)
    mid = (F(n) + F(1, 2)) ** 2
    if t > mid or (t == mid and n % 2 == 1):
        n += 1
    return n * ulp


def from_bits(u: int) -> Fraction:
    return F(struct.unpack("<f", struct.pack("<I", u))[0])


def to_bits(q) -> int:
    return struct.unpack("<I", struct.pack("<f", float(q)))[0]


# ----------------------------------------------------- float32 literals ----

LITERALS = {  # Go source text -> float32 bits
    "1.442695041": 0x3FB8AA3B,
    "0.693147180559945": 0x3F317218,
    "0.240226506959101": 0x3E75FDF0,
    "0.055504108664821": 0x3D635847,
    "0.009676036358193": 0x3C1E883D,
    "22026.4657948": 0x46AC14EE,
    "1.702": 0x3FD9DB23,
    "1e-6": 0x358637BD,
}
LOG2E = from_bits(0x3FB8AA3B)
COEF = tuple(from_bits(u) for u in (0x3F317218, 0x3E75FDF0, 0x3D635847, 0x3C1E883D))
# The polynomial as the comment above it prints it (activation.go:117): a plausible
# restatement mistake, not the constants the code uses.
COEF_6DIGIT = tuple(r32(F(s)) for s in ("0.693147", "0.240227", "0.055504", "0.009676"))
EXP10 = from_bits(0x46AC14EE)
SCALE = from_bits(0x3FD9DB23)
EPS = from_bits(0x358637BD)


# --------------------------------------------------- models with knobs ----

def model_fast_exp(x, trunc=True, coef=COEF, horner="f32", log2e=LOG2E, clamp_le=False):
    """fastExp, activation.go:100-145.  Knobs: trunc (int32(y) toward zero, or
    floor), coef, horner ("f32": eight roundings; "fma": four fused steps;
    "f64": the polynomial in float64, rounded once), clamp_le (x <= -10 -> 0)."""
    x = F(x)
    if x < -10 or (clamp_le and x == -10):
        return F(0)
    if x > 10:
        return EXP10
    y = r32(x * log2e)
    i = int(y) if trunc else math.floor(y)
    f = r32(y - i)
    c1, c2, c3, c4 = coef
    if horner == "f32":
        t = r32(c3 + r32(f * c4))
        t = r32(c2 + r32(f * t))
        t = r32(c1 + r32(f * t))
        poly = r32(1 + r32(f * t))
    elif horner == "fma":
        t = r32(c3 + f * c4)
        t = r32(c2 + f * t)
        t = r32(c1 + f * t)
        poly = r32(1 + f * t)
    else:
        t = r64(c3 + r64(f * c4))
        t = r64(c2 + r64(f * t))
        t = r64(c1 + r64(f * t))
        poly = r32(r64(1 + r64(f * t)))
    if -126 <= i <= 127:
        return r32(poly * F(2) ** i)
    return F(0) if i < -126 else r32(F("3.402823e+38"))


def model_gelu(x, branches="ref", scale_f64=False, **exp_knobs):
    """GELUQuickSIMD, activation.go:47-95.  branches: "ref" (two branches on
    the sign of sx), "pos_only" (1/(1+fastExp(-sx)) everywhere), "neg_only"
    (e/(1+e) everywhere); scale_f64: sx from the double 1.702 * x."""
    x = F(x)
    sx = r32(F("1.702") * x) if scale_f64 else r32(SCALE * x)
    pos = sx >= 0 if branches == "ref" else branches == "pos_only"
    if pos:
        sig = r32(1 / r32(1 + model_fast_exp(-sx, **exp_knobs)))
    else:
        e = model_fast_exp(sx, **exp_knobs)
        sig = r32(e / r32(1 + e))
    return r32(x * sig)


def model_softmax(xs, group="ref", norm="recip", **exp_knobs):
    """Softmax, activation.go:161-213.  group: "ref" sum + (((e0+e1)+e2)+e3),
    "serial" ((((sum+e0)+e1)+e2)+e3), "pairs" sum + ((e0+e1)+(e2+e3));
    norm: "recip" (e * (1/sum)) or "div" (e / sum)."""
    xs = [F(v) for v in xs]
    mx = max(xs)
    es = [model_fast_exp(r32(v - mx), **exp_knobs) for v in xs]
    s, i, n = F(0), 0, len(es)
    while i + 3 < n:
        e0, e1, e2, e3 = es[i:i + 4]
        if group == "ref":
            s = r32(s + r32(r32(r32(e0 + e1) + e2) + e3))
        elif group == "serial":
            s = r32(r32(r32(r32(s + e0) + e1) + e2) + e3)
        else:
            s = r32(s + r32(r32(e0 + e1) + r32(e2 + e3)))
        i += 4
    for e in es[i:]:
        s = r32(s + e)
    if norm == "recip":
        inv = r32(1 / s)
        return [r32(e * inv) for e in es]
    return [r32(e / s) for e in es]


def model_rmsnorm(x, w, eps=EPS, order="ref", rms="two", mean="div"):
    """RMSNorm, norm.go:8-36 with the AVX2 sum of squares.  order: "ref"
    (x*inv)*w, "fold_w" x*(inv*w); rms: "two" (float32(sqrt(float64)) then
    1/rms) or "one" (float32 of the double 1/sqrt); mean: "div" (sumSq/n) or
    "recip" (sumSq*(1/n))."""
    n = len(x)
    lanes = [F(0)] * 8
    n8 = n & ~7
    for i in range(0, n8, 8):
        for v in range(8):
            lanes[v] = r32(x[i + v] * x[i + v] + lanes[v])
    ln = lanes
    ss = r32(r32(r32(ln[0] + ln[4]) + r32(ln[1] + ln[5])) + r32(r32(ln[2] + ln[6]) + r32(ln[3] + ln[7])))
    for i in range(n8, n):
        ss = r32(ss + r32(x[i] * x[i]))
    ms = r32(ss / n) if mean == "div" else r32(ss * r32(F(1, n)))
    a = r32(ms + eps)
    if rms == "two":
        inv = r32(1 / r32(sqrt_rnd(a, 53)))
    else:
        inv = r32(r64(1 / sqrt_rnd(a, 80)))
    if order == "ref":
        return [r32(r32(xi * inv) * wi) for xi, wi in zip(x, w)]
    return [r32(xi * r32(inv * wi)) for xi, wi in zip(x, w)]


def model_rope(v0, v1, c, s, fuse=None):
    """The rotation of one pair, rope_cache.go:102-103.  fuse: None (four
    rounded products), "x0_first" fma(v0, c, -v1*s), "x0_second"
    fma(-v1, s, v0*c), "x1_first" fma(v0, s, v1*c), "x1_second"
    fma(v1, c, v0*s)."""
    v0, v1, c, s = F(v0), F(v1), F(c), F(s)
    a, b, cc, d = r32(v0 * c), r32(v1 * s), r32(v0 * s), r32(v1 * c)
    x0 = r32(a - b)
    x1 = r32(cc + d)
    if fuse == "x0_first":
        x0 = r32(v0 * c - b)
    elif fuse == "x0_second":
        x0 = r32(a - v1 * s)
    elif fuse == "x1_first":
        x1 = r32(v0 * s + d)
    elif fuse == "x1_second":
        x1 = r32(cc + v1 * c)
    return x0, x1


# ------------------------------------------------------------------ pins ----

@dataclasses.dataclass(frozen=True)
class Pin:
    name: str
    fn: str            # "fast_exp" | "gelu" | "softmax" | "rmsnorm" | "rope"
    inputs: tuple      # float32 bit patterns (see each kind below)
    expected: tuple    # float32 bit patterns of the outputs
    doc: str


P = 1 + F(1, 2 ** 23)   # 0x3F800001
Q = 1 + F(1, 2 ** 22)   # 0x3F800002
H = F(1, 2)

RMS_N = 768

PINS = (
    Pin("fast_exp_trunc_half", "fast_exp", (0xBEB17218,), (0x3F3507C4,),
        """x = 0xBEB17218 (-0.34657359...), chosen so that y = x*log2e rounds to -0.5
        exactly (0xBF000000).  int32(y) = 0 (toward zero), f = y - 0 = -0.5.  Every
        product by f is a power-of-two scaling, so only the four additions round:
          f*c4 = -10389565*2^-31;  c3 + f*c4 = (119194168 - 10389565)*2^-31
               = 13600575.375 * 2^-28 -> 13600575*2^-28 (0x3D4F873F, ulp 2^-28);
          f*t  = -13600575*2^-29;  c2 + f*t = (16121328 - 1700071.875)*2^-26
               = 14421256.125*2^-26 -> 14421256*2^-26 (0x3E5C0D08);
          f*t  = -1802657*2^-24;   c1 + f*t = 9826423*2^-24 exactly (0x3F15F077);
          f*t  = -9826423*2^-25;   1 + f*t = 23728009*2^-25 = 11864004.5*2^-24, a tie,
               to even: 11864004*2^-24 = 0x3F3507C4.
        2^0 leaves it: fastExp = 0x3F3507C4 (0.70714974).  With floor(y) = -1 instead,
        f = +0.5 and the result is 0x3F35039F; with the comment's 6-digit coefficients
        0x3F3507C8; with the polynomial in float64 the final tie is not a tie:
        0x3F3507C5."""),
    Pin("fast_exp_trunc_neg", "fast_exp", (0xBF880000,), (0x3EB0F51D,),
        """x = -1.0625.  y = fl(-1.0625 * 12102203*2^-23) = 0xBFC434DF (-1.53286350);
        int32(y) = -1, f = y + 1 = 0xBF0869BE (-0.53286350, exact), poly = 0x3F30F51D,
        times 2^-1: 0x3EB0F51D.  floor: 0x3EB0F056; 6-digit coefficients: 0x3EB0F520;
        fused Horner steps: 0x3EB0F51C; float64 polynomial: 0x3EB0F51C."""),
    Pin("fast_exp_log2e_rounding", "fast_exp", (0xC0280000,), (0x3D9474EC,),
        """x = -2.625.  With the float32 log2e, y = fl(-2.625 * 12102203*2^-23) =
        0xC0725F6D (-3.78707433; the exact product is -31768282.875*2^-23, ulp 2^-22 in
        this binade: -15884141.4375*2^-22 -> -15884141*2^-22); i = -3, f = 0xBF497DB4
        (-0.78707433), result 0x3D9474EC (0.07248864).  The float64 log2e would give
        y = 0xC0725F6E and 0x3D9474EB; floor 0x3D945B49; 6-digit coefficients
        0x3D9474F5; fused Horner and float64 polynomial 0x3D9474ED."""),
    Pin("fast_exp_pos", "fast_exp", (0x40000000,), (0x40EC59E0,),
        """x = 2.  y = 0x4038AA3B (2.88539004), i = 2, f = 0x3F62A8EC (0.88539004),
        poly = 0x3FEC59E0, times 4: 0x40EC59E0 (7.38597107).  6-digit coefficients:
        0x40EC59E2; fused Horner: 0x40EC59E1; float64 polynomial: 0x40EC59E1."""),
    Pin("fast_exp_clamp_edge", "fast_exp", (0xC1200000, 0xC1200001, 0x41200000, 0x41200001),
        (0x383E6D1C, 0x00000000, 0x46AC1458, 0x46AC14EE),
        """x = -10 is not clamped (the test is x < -10): y = 0xC166D4CA, i = -14,
        f = 0xBEDA9940, poly = 0x3F3E6D1C, result 0x383E6D1C (4.5401146e-5).  The
        next float below -10 gives 0.  x = 10: y = 0x4166D4CA, i = 14, poly 0x3FAC1458,
        0x46AC1458 (22026.172); the next float above 10 returns the literal
        22026.4657948 = 0x46AC14EE."""),
    Pin("gelu_negative_branch", "gelu", (0xC0B40000,), (0xB9CD33C4,),
        """x = -5.625.  sx = fl(0x3FD9DB23 * -5.625) = 0xC1192E15 (-9.5737505); from the
        double 1.702 it would be 0xC1192E14.  sx < 0: e = fastExp(sx) = 0x3891EE86,
        1 + e = 0x3F800248, sigmoid = e / (1+e) = 0x3891EBEC, x * sigmoid = 0xB9CD33C4.
        The positive branch's form 1/(1+fastExp(-sx)) here gives 0xB9CD189A; the
        double 1.702 gives 0xB9CD33CC; floor in fastExp 0xB9CD09D5; 6-digit
        coefficients 0xB9CD33D2."""),
    Pin("gelu_positive_branch", "gelu", (0x3F000000,), (0x3EB3661A,),
        """x = 0.5.  sx = 0x3F59DB23 (0.851).  sx >= 0: e = fastExp(-sx) = 0x3EDA9E32,
        1 + e = 0x3FB6A78C, sigmoid = 1/(1+e) = 0x3F33661A, x * sigmoid = 0x3EB3661A
        (a halving).  The negative branch's form e/(1+e) with e = fastExp(sx) gives
        0x3EB3661B; 6-digit coefficients and fused Horner steps 0x3EB36619."""),
    Pin("softmax_group_order", "softmax",
        tuple(to_bits(v) for v in (0.0, -5.875, -4.25, -3.125, -5.375, -6.875, -2.0, -2.125)),
        (0x3F41B385, 0x3B0B49A8, 0x3C30D4FE, 0x3D082DE4, 0x3B65C256, 0x3A4D4688, 0x3DD1FC3F, 0x3DB91313),
        """n = 8, max 0.  e_i = fastExp(x_i) = 0x3F800000, 0x3B3815FA, 0x3C69B489,
        0x3D33FA46 | 0x3B97D3D4, 0x3A87A5FE, 0x3E0AC2BE, 0x3DF49945.  Group sums
        ((e0+e1)+e2)+e3 = 0x3F87CF46 and ((e4+e5)+e6)+e7 = 0x3E856EA6; sum = 0 + g1 + g2
        = 0x3FA92AF0.  Accumulated one by one, or as (e0+e1)+(e2+e3), the sum rounds to
        0x3FA92AEF and every p_i moves up one ulp (p_0 = 0x3F41B386).  1/sum = 0x3F41B385;
        p_i = e_i * (1/sum) as listed.  Dividing by the sum instead gives p_1 =
        0x3B0B49A9."""),
    Pin("rmsnorm_two_roundings", "rmsnorm", (7, 5, 65), (0x41373984, 0x4180DC7E),
        """n = 768, x = (7, 5, 0, ..., 0), w = (65/128, 1, 1, ...), eps = 0x358637BD.
        Lanes 0 and 1 hold 49 and 25; sumSq = 74 exactly.  meanSq = fl(74/768) =
        0x3DC55555 (74*(1/768 = 0x3AAAAAAB) would round to 0x3DC55556);
        meanSq + eps = 0x3DC555DB; sqrt in float64 then float32: rms = 0x3E9EEE3A;
        invRms = 1/rms = 0x404E2D97 (the double 1/sqrt rounded once: 0x404E2D96).
        y_0 = fl(fl(7 * invRms) * 65/128) = fl(0x41B467E4 * 65/128) = 0x41373984,
        y_1 = fl(5 * invRms) * 1 = 0x4180DC7E.  x*(invRms*w) instead: y_0 = 0x41373983
        (invRms*w = 0x3FD1664D); meanSq by the reciprocal: y_0 = 0x41373982; the
        one-rounding invRms: y_0 = 0x41373983."""),
    Pin("rope_unfused", "rope",
        # (v0, v1, cos, sin) per pair, as exact rationals
        ((P, 1, P * H, Q * H), (1, P, Q * H, P * H), (P, -1, Q * H, P * H), (-1, P, P * H, Q * H)),
        (0x00000000, 0x00000000, 0x3F800002, 0xBF800002, 0x3F800002, 0x3F800002, 0x00000000, 0x00000000),
        """Four pairs (i, i+half), with P = 1+2^-23 and Q = 1+2^-22 (cos and sin
        halved so they stay in [-1, 1]; the halving is exact):
          pair 0: v0 = P, v1 = 1, cos = P/2, sin = Q/2.  v0*cos = (1 + 2^-22 + 2^-46)/2
            rounds to Q/2 and v1*sin = Q/2, so x0' = 0.  Fusing v0*cos into the
            subtraction keeps 2^-47.  x1' = fl(P*Q/2) + P/2 = (1+3*2^-23)/2 + P/2 = Q
            exactly (0x3F800002).
          pair 1: v0 = 1, v1 = P, cos = Q/2, sin = P/2.  x0' = Q/2 - fl(P*P/2) = 0;
            fusing v1*sin gives -2^-47.  x1' = P/2 + fl(P*Q/2) = Q.
          pair 2: v0 = P, v1 = -1, cos = Q/2, sin = P/2.  x0' = fl(P*Q/2) + P/2 = Q;
            x1' = fl(P*P/2) - Q/2 = 0, fusing v0*sin gives 2^-47.
          pair 3: v0 = -1, v1 = P, cos = P/2, sin = Q/2.  x0' = -P/2 - fl(P*Q/2) = -Q;
            x1' = -Q/2 + fl(P*P/2) = 0, fusing v1*cos gives 2^-47.
        Outputs in memory order: x0' of pairs 0..3, then x1' of pairs 0..3."""),
)

# The knobs a restatement could plausibly get wrong, per function.
MUTANTS = {
    "fast_exp": {"floor": dict(trunc=False), "coef_6digit": dict(coef=COEF_6DIGIT),
                 "fused_horner": dict(horner="fma"), "f64_poly": dict(horner="f64"),
                 "clamp_le": dict(clamp_le=True), "log2e_f64": dict(log2e=F("1.442695040888963407"))},
    "gelu": {"pos_only": dict(branches="pos_only"), "neg_only": dict(branches="neg_only"),
             "scale_f64": dict(scale_f64=True), "floor": dict(trunc=False), "coef_6digit": dict(coef=COEF_6DIGIT)},
    "softmax": {"serial_sum": dict(group="serial"), "pairwise_sum": dict(group="pairs"), "divide": dict(norm="div"),
                "floor": dict(trunc=False)},
    "rmsnorm": {"fold_w": dict(order="fold_w"), "one_rounding_rsqrt": dict(rms="one"),
                "mean_by_reciprocal": dict(mean="recip")},
    "rope": {f: dict(fuse=f) for f in ("x0_first", "x0_second", "x1_first", "x1_second")},
}


def rmsnorm_operands(pin: Pin):
    """(x [768], w [768]) of an RMSNorm pin as exact rationals."""
    a, b, wnum = pin.inputs
    x = [F(0)] * RMS_N
    x[0], x[1] = F(a), F(b)
    w = [F(1)] * RMS_N
    w[0] = F(wnum, 128)
    return x, w


def model_eval(pin: Pin, **knobs):
    """The pin's outputs under the model with the given knobs, as bit patterns."""
    if pin.fn == "fast_exp":
        return tuple(to_bits(model_fast_exp(from_bits(u), **knobs)) for u in pin.inputs)
    if pin.fn == "gelu":
        return tuple(to_bits(model_gelu(from_bits(u), **knobs)) for u in pin.inputs)
    if pin.fn == "softmax":
        return tuple(to_bits(v) for v in model_softmax([from_bits(u) for u in pin.inputs], **knobs))
    if pin.fn == "rmsnorm":
        x, w = rmsnorm_operands(pin)
        return tuple(to_bits(v) for v in model_rmsnorm(x, w, **knobs)[:2])
    if pin.fn == "rope":
        outs = [model_rope(*pair, **knobs) for pair in pin.inputs]
        return tuple(to_bits(o[0]) for o in outs) + tuple(to_bits(o[1]) for o in outs)
    raise ValueError(pin.fn)
