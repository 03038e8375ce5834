"""CPU checks of the exponential that every three-centre node loop runs on the device (common.h
exp_cubic, exp_neg_tab_k, exp_neg_tab_k_w).

The constants are read from the source, and each function's instruction sequence is replayed in
doubles. Every fma is rounded once, from exact rationals. The integer steps are replayed on the
bit patterns. The results are compared with mpmath's e^x at 40 digits. The cubic is the minimax
fit of the relative error on the reduced range, so its error must equioscillate at its bound.
A wrong scale K, a dropped coefficient or a misplaced table shift fails these bounds by orders of
magnitude.
"""
import math
import re
import struct
from fractions import Fraction

import mpmath as mp
import numpy as np

from conftest import ROOT

mp.mp.dps = 40
SRC = (ROOT / "gs-dft_amd" / "csrc" / "common.h").read_text()


def _const(name):
    m = re.search(rf"constexpr double {name} = (-?0x[0-9a-fA-F.]+p[+-]?\d+);", SRC)
    assert m, name
    return float.fromhex(m.group(1))


K, A2, A1, A0 = (_const(n) for n in ("kExpPolyK", "kExpA2", "kExpA1", "kExpA0"))
C256 = _const("kNegC256")
CAP_W = float(re.search(r"constexpr double kFoldCapZ = ([0-9.]+);", SRC).group(1))
MIN_EXP = int(re.search(r"constexpr int kFoldMinExp = (-?\d+);", SRC).group(1))
LN2_256 = {float.fromhex(v) for v in re.findall(r"__builtin_fma\(-kf, (0x[0-9a-f.]+p-9), -z\)", SRC)}
TAB = [float.fromhex(v.strip()) for v in
       re.search(r"exp2_frac\(int j\) \{\s*constexpr double t\[256\] = \{(.*?)\};", SRC,
                 re.S).group(1).split(",") if v.strip()]
SHIFT = float.fromhex("0x1.8p52")
H = math.log(2) / 512


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def _bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def _double(u):
    return struct.unpack("<d", struct.pack("<Q", u & (2 ** 64 - 1)))[0]


def exp_cubic(r):
    p = r + A2
    p = fma(p, r, A1)
    return fma(p, r, A0)


def _tab_scale(sh, p):
    """lead[k & 255] with k << 12 added to its high word, times p (k: the low word of sh)."""
    k = _bits(sh) & 0xFFFFFFFF
    j = k & 255
    lead = _bits(TAB[j]) - (j << 44)
    hi = ((lead >> 32) + ((k << 12) & 0xFFFFFFFF)) & 0xFFFFFFFF
    return _double((hi << 32) | (lead & 0xFFFFFFFF)) * p


def exp_neg_tab_k(z):
    (ln2_256,) = LN2_256
    z = min(z, 708.3)
    sh = fma(z, C256, SHIFT)
    kf = sh - SHIFT
    r = fma(-kf, ln2_256, -z)
    return _tab_scale(sh, exp_cubic(r))


def fold_weight(wh):
    n = max(int(np.rint(math.log2(wh))), MIN_EXP)
    return -math.log(math.ldexp(wh, -n)), SHIFT + 256.0 * n


def exp_neg_tab_k_w(z, S):
    (ln2_256,) = LN2_256
    z = min(z, CAP_W)
    sh = fma(z, C256, S)
    kf = sh - S
    r = fma(-kf, ln2_256, -z)
    return _tab_scale(sh, exp_cubic(r))


def _rel(v, ref):
    return float(mp.mpf(v) / ref - 1)


def test_constants_parsed():
    assert len(TAB) == 256 and len(LN2_256) == 1
    assert TAB[0] == 1.0
    assert all(abs(_rel(TAB[j], mp.mpf(2) ** (mp.mpf(j) / 256))) < 1.2e-16 for j in range(256))
    assert abs(_rel(next(iter(LN2_256)), mp.log(2) / 256)) < 1.2e-16
    assert abs(_rel(-C256, 256 / mp.log(2))) < 1.2e-16


def test_cubic_is_the_minimax_fit_of_k_e_r():
    """|p(r) / (K e^r) - 1| <= 2.05e-14 on |r| <= ln2/512, reaching nearly that bound with both
    signs (the equioscillation of a minimax fit: a scale K off by one part in 1e13 breaks it)."""
    rs = np.linspace(-H * (1 + 1e-6), H * (1 + 1e-6), 2001)
    err = np.array([_rel(exp_cubic(float(r)), mp.mpf(K) * mp.e ** mp.mpf(float(r))) for r in rs])
    assert np.max(np.abs(err)) < 2.05e-14
    assert np.max(err) > 1.5e-14 and np.min(err) < -1.5e-14
    assert abs(np.mean(err)) < 3e-15


def test_table_exp_relative_error():
    """exp_neg_tab_k(z) = K e^-z over z in [-1, 708.3] within the cubic's 2.05e-14 plus z d
    relative, d the relative error of ln2/256 as one double (3.3e-17: the reduction's error grows
    with z, while e^-z itself shrinks); beyond the cap it returns the capped value (normal,
    positive)."""
    (ln2_256,) = LN2_256
    d = abs(float((mp.mpf(ln2_256) - mp.log(2) / 256) / (mp.log(2) / 256)))
    rng = np.random.default_rng(7)
    zs = np.concatenate([rng.uniform(-1, 1, 300), rng.uniform(1, 60, 600),
                         rng.uniform(60, 708.3, 100), [0.0, -1.0, 36.0, 708.3]])
    err = np.array([_rel(exp_neg_tab_k(float(z)), mp.mpf(K) * mp.e ** (-mp.mpf(float(z))))
                    for z in zs])
    assert np.all(np.abs(err) < 2.05e-14 + np.abs(zs) * d + 4e-16)
    assert np.max(np.abs(err[zs <= 60])) < 2.3e-14
    capped = exp_neg_tab_k(708.3)
    assert exp_neg_tab_k(1e4) == capped and capped > 2.2e-308


def test_folded_weight_exp_relative_error():
    """exp_neg_tab_k_w(z - ln w', S) = K wh e^-z for wh = 2^n w' (fold_weight), weights from
    1e-18 to 1e3 (below 2^kFoldMinExp the rest of the weight stays in w')."""
    rng = np.random.default_rng(11)
    for wh in np.concatenate([10.0 ** rng.uniform(-18, 3, 60), [1.0, 0.5, 2.0 ** MIN_EXP / 3]]):
        lw, S = fold_weight(float(wh))
        assert abs(lw) <= math.log(2) / 2 + 1e-15 or wh < 2.0 ** MIN_EXP
        for z in rng.uniform(-1, 40, 20):
            ref = mp.mpf(K) * mp.mpf(float(wh)) * mp.e ** (-mp.mpf(float(z)))
            got = exp_neg_tab_k_w(float(z) + lw, S)
            # z + lw rounds to one double: ~|z| 2^-53 of relative error on top of the cubic's
            assert abs(_rel(got, ref)) < 2.5e-14 + abs(float(z)) * 2.3e-16, (wh, z)
