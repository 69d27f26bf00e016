"""Pins the float64 attention reference of the fused-kernel tests by closed forms
(no reference test checks attention outputs): two-token logistic weights with the
1/sqrt(d) scale, uniform keys giving the mean of V, a dominant key selecting its V
row, the grouped-query head mapping, and scipy's softmax on random inputs."""

import numpy as np
from scipy.special import softmax

from attention_ref import attention_f64


def test_two_tokens_give_logistic_weights_with_sqrt_d_scale():
    d = 128
    q = np.zeros((1, d))
    q[0, 0] = 3.0
    k = np.zeros((2, 1, d))
    k[0, 0, 0], k[1, 0, 0] = 2.0, -1.0
    v = np.zeros((2, 1, d))
    v[0, 0, :] = 1.0
    v[1, 0, :] = -2.0
    # s0 - s1 = 3 * (2 - (-1)) / sqrt(128)
    p0 = 1.0 / (1.0 + np.exp(-9.0 / np.sqrt(d)))
    want = p0 * 1.0 + (1 - p0) * -2.0
    np.testing.assert_allclose(attention_f64(q, k, v)[0], want, rtol=1e-13)


def test_uniform_keys_average_the_values():
    rng = np.random.default_rng(0)
    k = np.tile(rng.normal(size=(1, 1, 64)), (37, 1, 1))
    v = rng.normal(size=(37, 1, 64))
    q = rng.normal(size=(1, 64))
    np.testing.assert_allclose(attention_f64(q, k, v)[0], v[:, 0].mean(axis=0), rtol=1e-12)


def test_dominant_key_selects_its_value_row():
    rng = np.random.default_rng(1)
    d = 128
    k = rng.normal(size=(50, 1, d)) * 0.01
    q = np.zeros((1, d))
    q[0, 5] = 40.0
    k[17, 0, 5] = 40.0  # score 1600 / sqrt(128) above the rest
    v = rng.normal(size=(50, 1, d))
    np.testing.assert_allclose(attention_f64(q, k, v)[0], v[17, 0], rtol=1e-12, atol=1e-12)


def test_grouped_query_heads_read_their_kv_head():
    rng = np.random.default_rng(2)
    kv_heads, group, d, t = 3, 4, 16, 9
    k = rng.normal(size=(t, kv_heads, d))
    v = rng.normal(size=(t, kv_heads, d))
    q = rng.normal(size=(kv_heads * group, d))
    got = attention_f64(q, k, v)
    for h in range(kv_heads * group):
        alone = attention_f64(q[h:h + 1], k[:, h // group:h // group + 1],
                              v[:, h // group:h // group + 1])
        np.testing.assert_allclose(got[h], alone[0], rtol=1e-13)


def test_matches_scipy_softmax_formula():
    rng = np.random.default_rng(3)
    kv_heads, group, d, t = 2, 4, 128, 300
    k = rng.normal(size=(t, kv_heads, d)) * 3
    v = rng.normal(size=(t, kv_heads, d))
    q = rng.normal(size=(kv_heads * group, d))
    got = attention_f64(q, k, v)
    for h in range(kv_heads * group):
        w = softmax(k[:, h // group] @ q[h] / np.sqrt(d))
        np.testing.assert_allclose(got[h], w @ v[:, h // group], rtol=1e-10, atol=1e-12)
