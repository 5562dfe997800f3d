"""The GPU quantizer's division-free path (device.h q8_value_fast), restated
in numpy float32 on the CPU: y = x * rcp(s), q = rint(y), and the correctly
rounded x / s wherever |y - q| >= 0.5 - 2^-13.  It must equal the
reference's rint(x / s) (runq.c:117-139) on every input, including inputs
a few ulps from the rounding boundaries (k + 1/2) * s, with rcp modelled as
1 ulp off in either direction.  The GPU kernel itself is checked against the
oracle in tests/test_gpu_ops.py."""
import numpy as np

F = np.float32


def fast_quantize(x, s, r):
    y = (x * r).astype(F)
    q = np.rint(y).astype(F)
    slow = ~(np.abs((y - q).astype(F)) < F(0.5) - F(2.0 ** -13))
    return np.where(slow, np.rint(np.clip((x / s).astype(F), F(-127), F(127))), q), slow


def test_fast_quantizer_equals_division():
    rng = np.random.default_rng(0)
    n, g = 1 << 20, 64
    amax = (np.abs(rng.standard_normal(n // g)) * 10.0 ** rng.integers(-6, 6, n // g)).astype(F)
    s = np.where(amax == 0, F(1e-8), (amax / F(127)).astype(F)).astype(F)
    S, A = np.repeat(s, g), np.repeat(amax, g)
    x = (rng.uniform(-1, 1, n).astype(F) * A).astype(F)
    k = rng.integers(-127, 127, n).astype(F) + F(0.5)
    near = (k * S).astype(F)
    for _ in range(3):
        step = rng.integers(-1, 2, n)
        near = np.where(step > 0, np.nextafter(near, F(np.inf)),
                        np.where(step < 0, np.nextafter(near, F(-np.inf)), near)).astype(F)
    pick = (rng.random(n) < 0.5) & (np.abs(near) <= A)
    x = np.where(pick, near, x).astype(F)
    exact = np.rint((x / S).astype(F))
    r0 = (F(1) / S).astype(F)
    for dirn in (-1, 0, 1):
        r = r0 if dirn == 0 else np.nextafter(r0, F(np.inf) if dirn > 0 else F(-np.inf)).astype(F)
        q, slow = fast_quantize(x, S, r)
        np.testing.assert_array_equal(q, exact)
        assert slow[pick].mean() > 0.5          # the guard does fire near the boundaries
        assert slow[~pick].mean() < 2e-3        # and almost never elsewhere
    assert np.abs(exact).max() <= 127           # the clamp of the reference never binds


def test_scale_fma_form_equals_division_exhaustively(tmp_path):
    """device.h q8_scale computes amax / 127 as s0 = amax * RN(1/127) plus one
    FMA correction; over every finite float amax >= 0 it must give the
    correctly rounded quotient of the reference (runq.c:117-139).  Built with
    gcc from tests/q8_scale_check.c (hardware or libm fmaf: both correctly
    rounded; no flush of denormals, as on the GPU)."""
    import os
    import subprocess
    src = os.path.join(os.path.dirname(__file__), "q8_scale_check.c")
    exe = str(tmp_path / "q8_scale_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", src, "-o", exe, "-lm"], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    assert int(out.strip()) == 0


def test_magic_add_rounding_equals_rint():
    """device.h q8_byte_fast rounds y (|y| < 128) by t = y + 1.5*2^23 in
    float32 and takes the int8 value from the low byte of t's bits.  That
    must be rint(y) (ties to even) as int8, at every half-integer and a few
    ulps around it, and on a dense sample of the range."""
    M = F(1.5 * 2 ** 23)
    k = np.arange(-128, 128, dtype=np.float64)
    y = [(k + 0.5).astype(F)]
    for _ in range(4):
        y.append(np.nextafter(y[-1], F(np.inf)))
    lo = [(k + 0.5).astype(F)]
    for _ in range(4):
        lo.append(np.nextafter(lo[-1], F(-np.inf)))
    rng = np.random.default_rng(5)
    y = np.concatenate(y + lo + [k.astype(F), rng.uniform(-128, 128, 1 << 22).astype(F)])
    y = y[np.abs(y) < 128]
    t = (y + M).astype(F)
    byte = (t.view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    q = np.rint(y).astype(np.int32)
    np.testing.assert_array_equal((t - M).astype(F), np.rint(y).astype(F))
    np.testing.assert_array_equal(byte.astype(np.int32), np.where(q > 127, q - 256, q))
