"""The device evaluates the reference's GELU (src/tensor.rs:289-305,
0.5 t (1 + tanh(z)), z = 0.7978846 (t + 0.044715 t^3)) as t / (1 + e^(-2z))
on the hardware's exp2 and reciprocal (rw_kernels.hpp, gelu).  Here that
form is evaluated in float32 with each operation rounded once (exp2 and the
reciprocal correctly rounded, as the hardware's are to within an ulp) and
checked against the tanh form in float64: the same function, within a few
float32 roundings everywhere, with the tanh form's special values."""
import numpy as np


def sigmoid_form_f32(t):
    t = np.asarray(t, np.float32)
    z = np.float32(0.7978846) * (t + np.float32(0.044715) * t * t * t)
    with np.errstate(over="ignore"):
        e = np.exp2((z * np.float32(-2.8853900817779268)).astype(np.float64)).astype(np.float32)
    with np.errstate(divide="ignore"):
        r = (1.0 / (np.float32(1.0) + e).astype(np.float64)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        return (t * r).astype(np.float32)


def tanh_form_f64(t):
    t = np.asarray(t, np.float64)
    z = 0.7978846 * (t + 0.044715 * t ** 3)
    return 0.5 * t * (1.0 + np.tanh(z))


def test_sigmoid_form_is_the_tanh_form():
    t = np.concatenate([np.linspace(-12, 12, 200001), np.random.default_rng(0).standard_normal(100000) * 4])
    got = sigmoid_form_f32(t.astype(np.float32)).astype(np.float64)
    want = tanh_form_f64(t.astype(np.float32))
    err = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
    ulp = 2.0 ** -24
    # where gelu is not small, a few roundings; in the negative tail, where
    # gelu(t) ~ t e^(-2|z|), the roundings of z are amplified by |2z| (<= 50
    # ulps down to |gelu| = 1e-6); never more than 1e-6 absolute
    assert np.max(err[np.abs(want) > 1e-2]) < 16 * ulp
    assert np.max(err[np.abs(want) > 1e-6]) < 64 * ulp
    assert np.max(np.abs(got - want)) < 1e-6
    # the tanh form itself in float32 loses more there (1 + tanh z cancels)
    t32 = t.astype(np.float32)
    z32 = np.float32(0.7978846) * (t32 + np.float32(0.044715) * t32 * t32 * t32)
    ref32 = (np.float32(0.5) * t32 * (np.float32(1.0) + np.tanh(z32))).astype(np.float64)
    tail = (np.abs(want) > 1e-6) & (t < -2)
    assert np.max(np.abs(ref32 - want)[tail] / np.abs(want[tail])) > np.max(err[tail])


def test_special_values():
    assert sigmoid_form_f32(np.float32(0.0)) == 0.0
    assert sigmoid_form_f32(np.float32(100.0)) == np.float32(100.0)
    neg = sigmoid_form_f32(np.float32(-100.0))
    assert neg == 0.0 and np.signbit(neg)
    assert sigmoid_form_f32(np.float32(np.inf)) == np.inf
    assert np.isnan(sigmoid_form_f32(np.float32(-np.inf)))
    assert np.isnan(sigmoid_form_f32(np.float32(np.nan)))
