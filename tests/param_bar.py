"""The parameter bar of the GPU parity tests, and the per-element error report they print.

The kernel's codes and block scales are compared bit for bit.  Its parameter update is not:
the oracle (as stquant_kernel.cu:136-143 with nvcc's IEEE defaults) computes
    den = RN(RN(RN(sqrt v) / D) + eps),  q = RN(m / den),  p' = RN(RN(p * decay) - RN(s * q))
with D = RN(sqrt bc2) and s = lr / bc1, while the kernel computes
    den = RN(sqrt_hw(v) * RN(1 / D) + eps),  q = RN(m * rcp_hw(den)),  p' = RN(RN(p * decay) - s * q)
(one fused multiply-add), where sqrt_hw and rcp_hw are gfx950's v_sqrt_f32 / v_rcp_f32, each
within 1 ulp (2^-23 relative) of the exact value on the normal range (measured on every float by
tests/test_gpu_math.py).  With u = 2^-24 and both sums of non-negative terms:
    |den_k / den_o - 1| <= 2u (sqrt_hw) + u (RN(1/D)) + u (RN sqrt) + u (RN /D) + 2u (two RN adds) = 7u
    |q_k / q_o - 1|     <= 7u + 2u (rcp_hw) + u (RN product) + u (RN quotient)            = 11u
    |p'_k - p'_o|       <= 11u |s q| + u |s q| (the oracle's RN product) + u |p'_k| + u |p'_o|
                         ~ 12u |update| + 2u |p'|,
to first order.  The bar adds headroom to both terms:
    |dp| <= 2^-20 |update| + 2^-22 |p'|      (2^-20 = 16u, 2^-22 = 4u)
per element, with |update| = |p'_o - p_prev| (weight decay moves p by lr * wd * |p|, covered by
the second term) and an absolute floor of FLT_MIN for results below the normal range.

So an element's error relative to |p'| exceeds 1e-6 only where 2^-20 |update| > (1e-6 - 2^-22)|p'|,
i.e. where the update is at least 0.8 |p'|: parameters the step carries through (or next to) zero.
The report gives the share of such elements and checks that every one of them is of that kind.
"""
import numpy as np

# every comparison of the session: (label, stats), printed by conftest.py at the session's end
RECORDS = []

UPDATE_TERM = 2.0 ** -20
PARAM_TERM = 2.0 ** -22
FLOOR = float(np.finfo(np.float32).tiny)


def param_error_stats(got, want, prev):
    """Per-element comparison of the kernel's params ``got`` with the oracle's ``want`` after one
    step from ``prev`` (all float32 arrays of one shape)."""
    g = np.asarray(got, np.float32).ravel()
    w = np.asarray(want, np.float32).ravel()
    pv = np.asarray(prev, np.float32).ravel()
    g64, w64 = g.astype(np.float64), w.astype(np.float64)
    err = np.abs(g64 - w64)
    upd = np.abs(w64 - pv.astype(np.float64))
    bar = UPDATE_TERM * upd + PARAM_TERM * np.abs(w64) + FLOOR
    # relative error where the oracle's p' is nonzero; a p' of exactly 0 (the step cancels p) has
    # no relative error, and its absolute error is reported on its own (it is held to the bar too)
    zero_want = (w64 == 0) & (err > 0)
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where((err == 0) | zero_want, 0.0, err / np.abs(w64))
    # ulp distance on the ordered integer line of float32 bit patterns
    gi = g.view(np.int32).astype(np.int64)
    wi = w.view(np.int32).astype(np.int64)
    gi = np.where(gi < 0, -(gi & 0x7fffffff), gi)
    wi = np.where(wi < 0, -(wi & 0x7fffffff), wi)
    ulps = np.abs(gi - wi)
    over = rel > 1e-6
    big = np.abs(w64) >= 1e-30
    n = g.size
    return dict(
        n=n,
        identical=float(np.mean(g.view(np.uint32) == w.view(np.uint32))) if n else 1.0,
        max_ulps=int(ulps.max()) if n else 0,
        rel_q50=float(np.quantile(rel, 0.5)) if n else 0.0,
        rel_q99=float(np.quantile(rel, 0.99)) if n else 0.0,
        rel_q999=float(np.quantile(rel, 0.999)) if n else 0.0,
        rel_max=float(rel.max()) if n else 0.0,
        share_rel_over_1e6=float(np.mean(over)) if n else 0.0,
        # the elements above 1e-6 relative: the smallest ratio update / |p'| among them
        # (implied by the bar wherever |p'| is well above FLT_MIN * 2^20)
        min_update_ratio_over=(float(np.min(upd[over & big] / np.abs(w64[over & big])))
                               if (over & big).any() else None),
        zero_target=int(np.count_nonzero(zero_want)),
        zero_target_max_abs=float(err[zero_want].max()) if zero_want.any() else 0.0,
        bar_use=float(np.max(err / bar)) if n else 0.0,
        worst=int(np.argmax(err / bar)) if n else -1,
    )


def format_stats(s, label=""):
    over = s["share_rel_over_1e6"]
    tail = (f"; above 1e-6 relative: {100 * over:.4f} % of elements, each with |update| >= "
            f"{s['min_update_ratio_over']:.2f} |p'|" if over else "; none above 1e-6 relative")
    zero = (f"; p' = 0 in the oracle with dp != 0: {s['zero_target']} elements, max |dp| "
            f"{s['zero_target_max_abs']:.2e}" if s["zero_target"] else "")
    return (f"params{(' ' + label) if label else ''}: {s['n']:,} elements, {100 * s['identical']:.3f} % bit-identical, "
            f"max {s['max_ulps']} ulp; |dp|/|p'| (p' != 0) median {s['rel_q50']:.2e}, 99 % {s['rel_q99']:.2e}, "
            f"99.9 % {s['rel_q999']:.2e}, max {s['rel_max']:.2e}{tail}{zero}; bar use {s['bar_use']:.3f}")


def assert_param_bar(got, want, prev, label="", quiet=False):
    """Assert |dp| <= 2^-20 |update| + 2^-22 |p'| (+ FLT_MIN) per element and print the report."""
    s = param_error_stats(got, want, prev)
    RECORDS.append((label, s))
    if not quiet:
        print(format_stats(s, label), flush=True)
    if s["bar_use"] > 1.0:
        i = s["worst"]
        g = np.asarray(got, np.float32).ravel()[i]
        w = np.asarray(want, np.float32).ravel()[i]
        pv = np.asarray(prev, np.float32).ravel()[i]
        raise AssertionError(f"{label} param {i}: got {g!r} want {w!r} prev {pv!r}: "
                             f"{s['bar_use']:.3f} x the bar 2^-20 |update| + 2^-22 |p'|")
    if s["min_update_ratio_over"] is not None:
        assert s["min_update_ratio_over"] >= 0.8, s
    return s
