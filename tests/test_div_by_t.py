"""The fp32 top-p kernel's division by the temperature (div_by_t in
graspo_amd/csrc/tokpath_common.h) restated in numpy: wherever its
multiply-and-check fast path accepts q = RN(x * RN(1/T)), q must equal the
IEEE quotient RN(x / T); every other token takes the division itself.

The restatement is exact: a product of two fp32 values is exact in fp64, so
RN32 of it is the fp32 multiply, and x - q T (q within 2 ulp of x / T) spans
under 53 bits, so RN32 of its fp64 value is the fma's single rounding.
Cases: temperatures log-uniform over [2^-20, 1024] and the usual ones,
logits over many magnitudes, and logits built so that x / T falls within a
few ulp of a rounding midpoint, where a wrong bound would show."""

import numpy as np

F32 = np.float32


def fast_path(x, T):
    """(accepted, q) of div_by_t for fp32 arrays x and scalar fp32 T."""
    rT = F32(F32(1.0) / T)
    bh = F32(F32(T * F32(2.0 ** -25)) * F32(1.0 - 2.0 ** -20))
    q0 = (x.astype(np.float64) * np.float64(rT)).astype(F32)
    r0 = (x.astype(np.float64) - q0.astype(np.float64) * np.float64(T)).astype(F32)
    # one correction, q = fma(r0, rT, q0) (its fp64 restatement may round
    # twice; the acceptance test below is exact for whatever q it gets)
    with np.errstate(invalid="ignore"):
        q = (q0.astype(np.float64) + r0.astype(np.float64) * np.float64(rT)).astype(F32)
    r = (x.astype(np.float64) - q.astype(np.float64) * np.float64(T)).astype(F32)
    with np.errstate(invalid="ignore", over="ignore"):
        _, e = np.frexp(q)
        h = np.ldexp(np.full(q.shape, bh, F32), e).astype(F32)
        ok = (np.abs(r) < h) & (e >= -59) & ((q.view(np.uint32) & 0x7FFFFF) != 0)
    return ok, q


def check(x, T):
    x = x.astype(F32)
    T = F32(T)
    ok, q = fast_path(x, T)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        want = (x / T).astype(F32)
    bad = ok & (q.view(np.uint32) != want.view(np.uint32))
    assert not bad.any(), (float(T), x[bad][:5], q[bad][:5], want[bad][:5])
    return ok.mean()


def temperatures(rng, n):
    t = np.exp2(rng.uniform(-20.0, 10.0, n)).astype(F32)
    return np.concatenate([t, np.array([0.7, 1.0, 0.6, 1.3, 2.0, 0.9, 1.5, 1e-6, 1024.0], F32)])


def test_fast_path_equals_the_ieee_quotient_on_random_logits():
    rng = np.random.default_rng(7)
    for T in temperatures(rng, 60):
        x = np.concatenate([
            rng.standard_normal(20000) * 3.0,
            rng.standard_normal(5000) * 3.0 + 1e-3 * rng.random(5000),
            np.exp2(rng.uniform(-80, 80, 5000)) * rng.choice([-1.0, 1.0], 5000),
            np.array([0.0, -0.0, 1.0, -1.0, 2.0 ** -60, 2.0 ** 100, np.inf, -np.inf, np.nan]),
        ])
        rate = check(x, T)
        assert rate > 0.95, (float(T), rate)  # the fast path is the common one


def test_fast_path_near_rounding_midpoints():
    """x chosen so that x / T lies within a few ulp(x / T) * 2^-20 of the
    midpoint between two fp32 values: the cases a loose bound would get wrong."""
    rng = np.random.default_rng(11)
    for T in temperatures(rng, 40):
        y = (rng.standard_normal(20000) * 8.0).astype(F32)
        y = y[(y != 0) & np.isfinite(y)]
        ulp = np.spacing(np.abs(y)).astype(np.float64)
        mid = y.astype(np.float64) + np.sign(y) * ulp / 2
        x = (mid * np.float64(T)).astype(F32)
        x = x[np.isfinite(x)]
        for k in (-2, -1, 1, 2):   # neighbours of each x as well
            check(np.nextafter(x, np.where(k > 0, np.inf, -np.inf).astype(F32)) if abs(k) == 1
                  else np.nextafter(np.nextafter(x, np.float32(np.inf * np.sign(k))),
                                    np.float32(np.inf * np.sign(k))), T)
        check(x, T)


def test_powers_of_two_and_tiny_quotients_take_the_division():
    T = F32(0.7)
    x = (np.exp2(np.arange(-30, 30, dtype=np.float64)) * np.float64(T)).astype(F32)
    ok, q = fast_path(x, T)
    assert not (ok & ((q.view(np.uint32) & 0x7FFFFF) == 0)).any()
    tiny = np.array([1e-30, -1e-25, 2.0 ** -70], F32)
    ok, _ = fast_path(tiny, F32(1.0))
    assert not ok.any()
