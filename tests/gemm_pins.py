"""Hand-derived vectors that pin the accumulation order of the Q8_0 x int8
GEMM, one output element each (batch 1, out_dim 1, two 32-wide blocks,
input scale 1).

The reference computes the element in one of four orders, chosen by the
build and the CPU:

- VNNI (internal/kernels/simd_amd64.s:241-304, picked on an AVX-512-VNNI host
  by simd_amd64.go:41-45): eight fp32 lanes; lane l accumulates the block sum
  over bytes 4l..4l+3 (VPDPBUSD, :279-288) with VCVTDQ2PS + VFMADD231PS
  (:290-291, one rounding per block); then the hsum
  ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) (:297-300).
- AVX2 (:164-237): the same, but lane l holds bytes 2l, 2l+1, 16+2l, 17+2l
  (VPMOVSXBW + VPMADDWD on each 16-byte half, VPADDD, :199-215).
- block-serial (matmul_inner_loop_fallback.go:16-43): one accumulator,
  acc = fma(P_b, d_b, acc) per block (as compiled on arm64, which fuses).
- arm64 assembly (simd_arm64_matmul.s:25-46): one accumulator, SCVTF, FMULS,
  FADDS: acc = acc + fl(P_b * d_b), two roundings per block.

Every value below is exact; the docstrings derive each order's result.  The
scales are fp16 values (the Q8_0 block scale), so powers of two and
1.5009765625 = 0x3E01 are exact.  In fp32, ulp(32768) = 2^-8, so adding 2^-10
to +-32768 rounds back to +-32768 (absorption); that is how a lane assignment
or a reduction tree shows in the result.
"""
from __future__ import annotations

import dataclasses
from fractions import Fraction

import numpy as np

ORDERS = ("vnni", "avx2", "block_serial", "arm64")

F = Fraction
P2_15 = F(2) ** 15
P2_M10 = F(1, 1024)


@dataclasses.dataclass(frozen=True)
class Pin:
    name: str
    doc: str
    scales: tuple          # per-block fp16-exact scale
    entries: tuple         # (block, byte, x, w) nonzero products
    expected: dict         # order -> exact Fraction

    def operands(self):
        """(x int8 [1, 64], w int8 [1, 64], d float16 [1, 2])."""
        nb = len(self.scales)
        x = np.zeros((1, 32 * nb), np.int8)
        w = np.zeros((1, 32 * nb), np.int8)
        for b, k, xv, wv in self.entries:
            x[0, 32 * b + k] = xv
            w[0, 32 * b + k] = wv
        d = np.array([[float(s) for s in self.scales]], np.float16)
        assert all(F(float(d[0, i])) == s for i, s in enumerate(self.scales)), "scale not exact in fp16"
        return x, w, d


PINS = (
    Pin("vnni_lanes",
        """Block 0 (d=2^15): +1 at byte 0, -1 at byte 16.  Block 1 (d=2^-10): +1 at byte 2.
        VNNI: bytes 0 and 2 share lane 0, byte 16 is lane 4.  Lane 0 = 2^15, lane 4 = -2^15;
        block 1 adds 2^-10 to lane 0, absorbed (2^15 + 2^-10 -> 2^15).  hsum: (2^15 - 2^15) = 0.
        AVX2: bytes 0 and 16 share lane 0, so block 0's lane sum is 1 - 1 = 0; byte 2 is lane 1
        = 2^-10; hsum = 2^-10.  Block-serial and arm64: P_0 = 0, P_1 = 1, result 2^-10.""",
        (P2_15, P2_M10), ((0, 0, 1, 1), (0, 16, 1, -1), (1, 2, 1, 1)),
        dict(vnni=F(0), avx2=P2_M10, block_serial=P2_M10, arm64=P2_M10)),
    Pin("avx2_lanes",
        """Block 0 (d=2^15): +1 at byte 0, -1 at byte 2.  Block 1 (d=2^-10): +1 at byte 16.
        AVX2: byte 0 and byte 16 are lane 0, byte 2 is lane 1.  Lane 0 = 2^15, lane 1 = -2^15;
        block 1's 2^-10 is absorbed into lane 0; hsum ((l0+l4)+(l1+l5)) = 2^15 - 2^15 = 0.
        VNNI: bytes 0 and 2 share lane 0 (1 - 1 = 0); byte 16 is lane 4 = 2^-10; hsum 2^-10.
        Block-serial and arm64: 2^-10.""",
        (P2_15, P2_M10), ((0, 0, 1, 1), (0, 2, 1, -1), (1, 16, 1, 1)),
        dict(vnni=P2_M10, avx2=F(0), block_serial=P2_M10, arm64=P2_M10)),
    Pin("vnni_hsum_tree",
        """Block 0 (d=2^15): +1 at byte 0 (VNNI lane 0), -1 at byte 16 (lane 4).  Block 1
        (d=2^-10): +1 at byte 4 (lane 1).  VNNI lanes: l0 = 2^15, l4 = -2^15, l1 = 2^-10.
        The reference tree adds l0+l4 = 0 before l1: ((l0+l4)+(l1+l5)) = 2^-10.  A serial
        l0+l1+...+l7 or an adjacent-pair tree ((l0+l1)+(l2+l3))+... adds l1 to 2^15 first
        and loses it: 0.  AVX2: bytes 0 and 16 cancel in lane 0, byte 4 is lane 2: 2^-10.
        Block-serial and arm64: 2^-10.""",
        (P2_15, P2_M10), ((0, 0, 1, 1), (0, 16, 1, -1), (1, 4, 1, 1)),
        dict(vnni=P2_M10, avx2=P2_M10, block_serial=P2_M10, arm64=P2_M10)),
    Pin("avx2_hsum_tree",
        """Block 0 (d=2^15): +1 at byte 0 (AVX2 lane 0), -1 at byte 8 (AVX2 lane 4).  Block 1
        (d=2^-10): +1 at byte 2 (AVX2 lane 1).  AVX2 lanes: l0 = 2^15, l4 = -2^15, l1 = 2^-10;
        the reference tree gives 2^-10, a serial or adjacent-pair tree 0.  VNNI: byte 0 and
        byte 2 are lane 0 (2^15, the 2^-10 absorbed), byte 8 is lane 2 (-2^15): 0.
        Block-serial and arm64: 2^-10.""",
        (P2_15, P2_M10), ((0, 0, 1, 1), (0, 8, 1, -1), (1, 2, 1, 1)),
        dict(vnni=F(0), avx2=P2_M10, block_serial=P2_M10, arm64=P2_M10)),
    Pin("arm64_unfused",
        """Block 0 (d=4): 127*-94 + 119*-1 = -12057 at bytes 0, 1; x4 = -48228 exactly.
        Block 1 (d=0x3E01=1.5009765625): 127*127 + 127*126 = 32131 at bytes 0, 1.
        Exact P_1*d_1 = 48196.5 + 32131/1024 = 48227.8779296875 (ulp 2^-8 at this size:
        224.75 ulps above 48227, so fl() = 48227.87890625).
        Fused (block-serial): fma(32131, d_1, -48228) = -0.1220703125 = -125/1024.
        Unfused (arm64): -48228 + 48227.87890625 = -0.12109375 = -124/1024.
        VNNI and AVX2: bytes 0 and 1 are lane 0 in both, so lane 0 runs the fused chain and
        the other lanes hold 0: -125/1024.""",
        (F(4), F(3, 2) + F(1, 1024)),
        ((0, 0, 127, -94), (0, 1, 119, -1), (1, 0, 127, 127), (1, 1, 127, 126)),
        dict(vnni=F(-125, 1024), avx2=F(-125, 1024), block_serial=F(-125, 1024), arm64=F(-124, 1024))),
    Pin("block_serial_fused",
        """As arm64_unfused, but block 1's products sit at bytes 4, 5 (VNNI lane 1, AVX2
        lane 2) while block 0 stays in lane 0.  Block-serial keeps one chain:
        fma(32131, d_1, -48228) = -125/1024.  arm64: -124/1024.  VNNI and AVX2: the lane
        holding block 1 starts from 0, so it rounds the product on its own to 48227.87890625,
        and the hsum adds -48228: -124/1024.""",
        (F(4), F(3, 2) + F(1, 1024)),
        ((0, 0, 127, -94), (0, 1, 119, -1), (1, 4, 127, 127), (1, 5, 127, 126)),
        dict(vnni=F(-124, 1024), avx2=F(-124, 1024), block_serial=F(-125, 1024), arm64=F(-124, 1024))),
)


# ---------------------------------------------------------------------------
# Exact-arithmetic model with knobs, used only to show that the vectors tell
# the four orders apart and catch a single mistake in any of them.  The pins
# themselves are the hand-derived `expected` values above.

def round_f32(q: Fraction) -> Fraction:
    """Round-to-nearest-even to float32 (normal and subnormal range)."""
    if q == 0:
        return F(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if F(2) ** e > a:
        e -= 1
    elif F(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = F(2) ** (e - 23)
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > F(1, 2) or (rem == F(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


LANE_MAPS = {
    "vnni": lambda k: k // 4,
    "avx2": lambda k: (k % 16) // 2,
    "single": lambda k: 0,
}


def _tree(lanes, kind):
    r = round_f32
    if kind == "avx":
        return r(r(r(lanes[0] + lanes[4]) + r(lanes[1] + lanes[5])) + r(r(lanes[2] + lanes[6]) + r(lanes[3] + lanes[7])))
    if kind == "pairs":
        return r(r(r(lanes[0] + lanes[1]) + r(lanes[2] + lanes[3])) + r(r(lanes[4] + lanes[5]) + r(lanes[6] + lanes[7])))
    s = lanes[0]
    for v in lanes[1:]:
        s = r(s + v)
    return s


def model(pin: Pin, lane_map: str, tree: str, fused: bool) -> Fraction:
    lanes = [F(0)] * 8
    lane_of = LANE_MAPS[lane_map]
    for b, d in enumerate(pin.scales):
        part = [0] * 8
        for bb, k, xv, wv in pin.entries:
            if bb == b:
                part[lane_of(k)] += xv * wv
        for l in range(8):
            if lane_map == "single" and l:
                continue
            if fused:
                lanes[l] = round_f32(part[l] * d + lanes[l])
            else:
                lanes[l] = round_f32(lanes[l] + round_f32(part[l] * d))
    return lanes[0] if lane_map == "single" else _tree(lanes, tree)


# The reference's configuration of each order.
CONFIG = {
    "vnni": ("vnni", "avx", True),
    "avx2": ("avx2", "avx", True),
    "block_serial": ("single", "avx", True),
    "arm64": ("single", "avx", False),
}
