"""CPU check of the soundness argument behind the LM head's int8 pre-pass (lm_head_q8_kernel in
flash_whisper_amd/csrc/decode.hip): with the kernel's quantization of the table and of y, its radius
r_v and its threshold rule, the row that wins the fp16-logit argmax (lowest index on ties) is always a
candidate. The fp32 logits are formed in two different summation orders (numpy's float32 matmul and a
pairwise float32 sum), and the argmax is taken over the fp16-rounded logits as the oracle does
(oracle.decoder.masked_argmax). Cases: random tables at several scales, planted ties, near-ties below
an fp16 ulp, y = 0, and logits past the fp16 range."""

import numpy as np

from oracle.decoder import masked_argmax

D = 1280
GAMMA = 7.7e-5  # >= D * 2^-24 / (1 - D * 2^-24), as in the kernel
YMAX = 127 * 128
ETA_PER_T = 0.51  # the kernel's bound on |y_i - t y_int_i| / t


def pack_table(w):
    """int8 rows, fp32 scales and fp32 error bounds, as lm_q8_pack_kernel builds them."""
    w = np.asarray(w, np.float32)
    amax = np.abs(w).max(1)
    s = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    q = np.clip(np.rint(w * inv[:, None]), -127, 127)
    err = np.sqrt(((w.astype(np.float64) - s[:, None].astype(np.float64) * q) ** 2).sum(1))
    e = np.nextafter(err.astype(np.float32), np.float32(np.inf))  # rounded up
    return q, s, e


def threshold(t):
    if not t > -65504.0:
        return -np.inf
    return min(t - (abs(t) * 2.0 ** -9 + 2.0 ** -23), 65504.0)


F32 = np.float32


def fma32(a, b, c):
    """fp32 fused multiply-add (the fp64 product of two fp32 values is exact; the sum is rounded to fp64,
    then to fp32: a double rounding that differs from one rounding only in rare ties)."""
    f64 = lambda x: np.asarray(x, F32).astype(np.float64)
    return (f64(a) * f64(b) + f64(c)).astype(F32)


def q8_step(amax, ysq):
    """The kernel's per-step constants (q8_step in flash_whisper_amd/csrc/decode_dev.h), in fp32."""
    t = F32(F32(amax) / F32(YMAX)) if amax > 0 else F32(1)
    ny = F32(F32(np.sqrt(F32(ysq))) * F32(1 + 2.0 ** -9))
    neta = F32(F32(F32(0.51) * t) * F32(35.77708764)) if amax > 0 else F32(0)
    k = fma32(GAMMA, ny, neta)
    return t, F32(ny + k), F32(k * F32(4543.6901))


def q8_bounds(ah, al, s, e, step, radius_scale=1.0, err_term=True):
    """The kernel's fp32 interval for a row's logit (q8_bounds in decode_dev.h), element-wise over rows;
    radius_scale = 0 plants the mistake of ranking by the estimate alone, err_term = False the mistake of
    leaving out the term that covers the fp32 rounding of the estimate."""
    t, a_e, b_s = step
    st = (np.asarray(s, F32) * t).astype(F32)
    fh = np.asarray(ah, np.float64).astype(F32)
    n = fma32(F32(128), fh, np.asarray(al, np.float64).astype(F32))
    av = (st * n).astype(F32)
    err = ((st * F32(2.0 ** -21)).astype(F32) * fma32(F32(128), np.abs(fh), np.abs(n))).astype(F32) * F32(err_term)
    inner = fma32(np.asarray(e, F32), a_e, (np.asarray(s, F32) * b_s).astype(F32))
    r = fma32(inner, F32(1 + 2.0 ** -18), (err + F32(1e-30)).astype(F32)) * F32(radius_scale)
    return (av + r).astype(F32), (av - r).astype(F32)


def candidates(q, s, e, y, live, radius_scale=1.0):
    y = np.asarray(y, np.float32)
    amax = np.abs(y).max()
    tinv = np.float32(YMAX / amax) if amax > 0 else np.float32(0)
    yi = np.clip(np.rint(y * tinv), -YMAX, YMAX)
    ysq = F32((y.astype(np.float64) ** 2).sum())
    hi = np.floor((yi + 64) / 128)                                  # the kernel's two digits
    lo = yi - 128 * hi
    ah, al = q @ hi, q @ lo                                         # exact integer dots
    ub, lb = q8_bounds(ah, al, s, e, q8_step(amax, ysq), radius_scale)
    ub = np.where(live, ub, -np.inf)
    lb = np.where(live, lb, -np.inf)
    thr = threshold(lb.max())
    return np.nonzero(live & ~(ub < thr))[0]


def fp16_argmax_two_orders(w, y, sup):
    w32, y32 = np.asarray(w, np.float32), np.asarray(y, np.float32)
    x1 = w32 @ y32                                                   # BLAS order
    x2 = (w32 * y32).reshape(len(w32), 32, 40).sum(2, dtype=np.float32).sum(1, dtype=np.float32)
    with np.errstate(over='ignore'):
        return [masked_argmax(np.float32(np.float16(x)), sup) for x in (x1, x2)]


def check(w, y, sup):
    q, s, e = pack_table(w)
    cand = set(candidates(q, s, e, y, ~sup).tolist())
    for win in fp16_argmax_two_orders(w, y, sup):
        assert win in cand, (win, len(cand))
    return len(cand)


def test_random_tables_all_scales():
    rng = np.random.default_rng(0)
    counts = []
    for trial in range(12):
        v = 2000
        w = np.float16(rng.standard_normal((v, D)) * 0.02 * (10.0 ** rng.uniform(-2, 1)))
        y = np.float16(rng.standard_normal(D) * (10.0 ** rng.uniform(-1, 1.5)))
        sup = rng.random(v) < 0.02
        counts.append(check(w, y, sup))
    assert max(counts) < 200  # the pre-pass does filter: a few rows of 2000, not all


def test_ties_near_ties_and_degenerate_inputs():
    rng = np.random.default_rng(1)
    w = np.float16(0.02 * rng.standard_normal((1500, D)))
    y = np.float16(rng.standard_normal(D))
    w[[10, 700, 1499]] = np.float16(0.05 * np.sign(y.astype(np.float32)))   # exact ties
    sup = np.zeros(1500, bool)
    check(w, y, sup)
    sup[10] = True
    check(w, y, sup)
    base = np.float16(0.03 * rng.standard_normal(D))                       # near-ties below one ulp
    for k in range(200, 400):
        r = base.copy()
        idx = rng.choice(D, 3, replace=False)
        r[idx] = np.nextafter(r[idx], np.float16(np.inf) if k % 2 else np.float16(-np.inf))
        w[k] = r
    check(w, np.float16(np.sign(base.astype(np.float32)) * np.abs(y.astype(np.float32))), np.zeros(1500, bool))
    assert check(w, np.zeros(D, np.float16), np.zeros(1500, bool)) == 1500  # y = 0: all rows tie
    big = np.full(D, 60000, np.float16)                                     # +-inf logits
    check(w, big, np.zeros(1500, bool))
    check(np.float16(np.full((300, D), -0.01)), big, np.zeros(300, bool))


def test_planted_mistake_is_caught():
    """Without the radius (ranking by the int8 estimate A_v alone) the winner escapes among near-tied
    rows, so the checks above would catch a radius that is too small."""
    rng = np.random.default_rng(2)
    sup = np.zeros(3000, bool)
    missed = 0
    for trial in range(10):
        w = np.float16(0.02 * rng.standard_normal((3000, D)))
        y = np.float16(rng.standard_normal(D))
        best = w[np.argmax(w.astype(np.float32) @ y.astype(np.float32))].astype(np.float64)
        w[:64] = np.float16(best + 1e-4 * rng.standard_normal((64, D)))  # 64 rows within a few fp16 ulps
        q, s, e = pack_table(w)
        win = fp16_argmax_two_orders(w, y, sup)[0]
        assert win in set(candidates(q, s, e, y, ~sup).tolist())
        missed += win not in set(candidates(q, s, e, y, ~sup, radius_scale=0.0).tolist())
    assert missed > 0


def _quantize_like_kernel(y):
    """t, y_int and eta = y - t y_int with the kernel's fp32 roundings (fp32 t and 1 / t, fp32 product,
    fused y - t y_int)."""
    y = np.asarray(y, np.float32)
    amax = np.abs(y).max()
    t = np.float32(amax / np.float32(YMAX))
    tinv = np.float32(np.float32(YMAX) / amax)
    yi = np.clip(np.rint(np.float32(y * tinv)), -YMAX, YMAX)
    eta = np.float32(y.astype(np.float64) - np.float64(t) * yi)
    return t, yi, eta


def test_eta_closed_form_bound_dominates():
    """|y_i - t y_int_i| <= 0.503 t for every element, so |eta| <= 0.51 t sqrt(1280), the bound the kernel
    uses instead of reducing |eta|^2: fp16 inputs over many scales, values at +-max |y|, and values one
    fp16 step either side of a half-integer multiple of t."""
    rng = np.random.default_rng(5)
    worst = 0.0
    for trial in range(400):
        scale = 10.0 ** rng.uniform(-4, 4)
        y = np.float16(rng.standard_normal(D) * scale)
        if trial % 4 == 1:  # heavy tails: a few large entries set max |y|
            y[rng.integers(0, D, 3)] = np.float16(min(scale * 40, 6e4))
        if trial % 4 == 2:  # entries near (k + 1/2) t
            amax = float(np.abs(y.astype(np.float32)).max())
            t = amax / YMAX
            k = rng.integers(-YMAX, YMAX, 64)
            y[:64] = np.float16((k + 0.5) * t)
            y[64:128] = np.float16(np.nextafter(np.float16((k + 0.5) * t), np.float16(np.inf)))
        if not np.isfinite(y.astype(np.float32)).all() or not np.abs(y).max() > 0:
            continue
        t, yi, eta = _quantize_like_kernel(y)
        per = np.abs(eta.astype(np.float64)) / np.float64(t)
        worst = max(worst, per.max())
        assert per.max() <= 0.503, per.max()
        assert np.sqrt((eta.astype(np.float64) ** 2).sum()) <= ETA_PER_T * np.float64(t) * np.sqrt(D)
    assert worst > 0.49  # the rounding errors do reach t / 2: the check is not vacuous


def test_fp32_interval_holds_the_exact_bound():
    """The kernel's fp32 interval [lb, ub] contains [A - r, A + r] with A = s t (128 ah + al) exact and r
    the radius of the soundness argument at its tightest: ||y|| <= sqrt(ysq) (1 + 2^-10) and
    ||eta|| <= 0.503 t sqrt(1280) (the bounds proved above and at q8_step). Random and adversarial values:
    digit dots at their extremes, 128 ah cancelling al, tiny and large scales, e = 0, y = 0."""
    from fractions import Fraction

    rng = np.random.default_rng(7)
    n_cases = 4000
    ah = rng.integers(-20_600_000, 20_600_000, n_cases)
    al = rng.integers(-10_400_000, 10_400_000, n_cases)
    ah[:500] = rng.integers(-81_000, 81_000, 500)          # 128 ah + al near 0
    al[:500] = -128 * ah[:500] + rng.integers(-3, 4, 500)
    ah[500:600], al[500:600] = 20_600_000, 10_400_000       # the extremes
    ah[600:700], al[600:700] = -20_600_000, -10_400_000
    s = F32(10.0 ** rng.uniform(-8, 0, n_cases))
    e = F32(s * F32(10.0 ** rng.uniform(-3, 1.6, n_cases)))
    e[700:800] = 0
    worst, escaped = np.inf, 0
    for i in range(n_cases):
        amax = F32(0) if i % 97 == 0 else F32(10.0 ** rng.uniform(-3, 4.5))
        ysq = F32(0) if amax == 0 else F32(amax * amax * rng.uniform(1, D))
        step = q8_step(amax, ysq)
        ub, lb = q8_bounds(np.array([ah[i]]), np.array([al[i]]), s[i:i + 1], e[i:i + 1], step)
        a_exact = Fraction(float(s[i])) * Fraction(float(step[0])) * (128 * int(ah[i]) + int(al[i]))
        ny = np.sqrt(np.float64(ysq)) * (1 + 2.0 ** -10)
        neta = 0.503 * np.float64(step[0]) * np.sqrt(D) if amax > 0 else 0.0
        r = (ny * np.float64(e[i]) + (neta + GAMMA * ny) * (127 * np.float64(s[i]) * np.sqrt(D) + np.float64(e[i])))
        r = Fraction(float(r * (1 + 1e-12)))
        assert Fraction(float(ub[0])) >= a_exact + r, i
        assert Fraction(float(lb[0])) <= a_exact - r, i
        if r > 0:
            worst = min(worst, float((Fraction(float(ub[0])) - a_exact) / r))
        ub0, lb0 = q8_bounds(np.array([ah[i]]), np.array([al[i]]), s[i:i + 1], e[i:i + 1], step, err_term=False)
        escaped += Fraction(float(ub0[0])) < a_exact + r or Fraction(float(lb0[0])) > a_exact - r
    assert escaped > 0  # without the rounding term the interval misses the exact one somewhere
    assert worst < 1.02  # and it is not wider than it needs to be by more than 2% (0.51 t against 0.503 t)
