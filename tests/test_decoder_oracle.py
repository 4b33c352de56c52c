"""Pins of the decoder oracle (CPU): properties the mathematics fixes, chosen so that a
plausible slip (interleaved instead of rotate-half RoPE pairs, a wrong sign, a kv-head index
off by the group, a causal mask off by one, a cache written at the wrong position) fails."""

import numpy as np
import pytest

import decoder_oracle as D


def test_rope_identity_at_zero_and_isometry():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 6, 64))
    assert np.allclose(D.rope(x, np.zeros(6), 1e4), x)
    y = D.rope(x, np.arange(6) * 37, 1e4)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))


def test_rope_rotates_half_pairs_at_the_published_frequencies():
    """Unit vector e_i (i < hd/2) at position p becomes cos(p w_i) e_i + sin(p w_i) e_{i+hd/2},
    w_i = base^(-2i/hd); e_{i+hd/2} becomes -sin e_i + cos e_{i+hd/2}."""
    hd, base, p = 64, 10000.0, 7
    for i in (0, 5, 31):
        w = base ** (-2.0 * i / hd)
        e = np.zeros((1, hd))
        e[0, i] = 1.0
        y = D.rope(e, np.array([p]), base)[0]
        want = np.zeros(hd)
        want[i], want[i + hd // 2] = np.cos(p * w), np.sin(p * w)
        assert np.allclose(y, want)
        e2 = np.zeros((1, hd))
        e2[0, i + hd // 2] = 1.0
        y2 = D.rope(e2, np.array([p]), base)[0]
        want2 = np.zeros(hd)
        want2[i], want2[i + hd // 2] = -np.sin(p * w), np.cos(p * w)
        assert np.allclose(y2, want2)


def test_rope_scores_depend_only_on_position_difference():
    rng = np.random.default_rng(1)
    q, k = rng.standard_normal((1, 128)), rng.standard_normal((1, 128))
    dots = [(D.rope(q, np.array([m + 5]), 1e4) @ D.rope(k, np.array([m]), 1e4).T)[0, 0] for m in (0, 3, 100, 999)]
    assert np.allclose(dots, dots[0])


def test_rmsnorm_has_unit_rms_for_unit_weights():
    rng = np.random.default_rng(2)
    h = rng.standard_normal((4, 256)) * 7.0
    out = D.rmsnorm(h, np.ones(256), 0.0)
    assert np.allclose(np.sqrt(np.mean(out * out, axis=-1)), 1.0)
    w = rng.standard_normal(256)
    assert np.allclose(D.rmsnorm(h, w, 0.0), out * w)


def test_attention_over_one_position_returns_v():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((4, 1, 64))
    k, v = rng.standard_normal((2, 1, 64)), rng.standard_normal((2, 1, 64))
    out = D.attention(q, k, v, np.array([0]))
    assert np.allclose(out, np.repeat(v, 2, axis=0))


def test_gqa_matches_loops_and_ignores_future_positions():
    """Brute force per head: q head h reads kv head h // (H / HK); positions past q_pos are masked."""
    rng = np.random.default_rng(4)
    H, HK, T, hd = 8, 2, 5, 16
    q = rng.standard_normal((H, T, hd))
    k, v = rng.standard_normal((HK, T, hd)), rng.standard_normal((HK, T, hd))
    pos = np.arange(T)
    out = D.attention(q, k, v, pos)
    for h in range(H):
        j = h // (H // HK)
        for t in range(T):
            s = np.array([q[h, t] @ k[j, u] / np.sqrt(hd) for u in range(t + 1)])
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[h, t], sum(p[u] * v[j, u] for u in range(t + 1)))
    k2, v2 = k.copy(), v.copy()
    k2[:, 3:], v2[:, 3:] = 1e3, -1e3  # future of query 2
    assert np.allclose(D.attention(q, k2, v2, pos)[:, :3], out[:, :3])


def _tiny_weights(rng, d=32, H=4, HK=2, hd=8, F=48, V=50, layers=2):
    def m(n, k):
        return rng.standard_normal((n, k)) / np.sqrt(k)
    layers_ = [D.OracleLayer(1 + 0.1 * rng.standard_normal(d), m((H + 2 * HK) * hd, d), m(d, H * hd),
                             1 + 0.1 * rng.standard_normal(d), m(2 * F, d), m(d, F)) for _ in range(layers)]
    w = D.OracleWeights(rng.standard_normal((V, d)), layers_, 1 + 0.1 * rng.standard_normal(d), m(V, d))
    return w, dict(heads=H, kv_heads=HK, head_dim=hd, ffn=F, eps=1e-5, rope_base=10000.0)


def test_prefill_equals_prefill_then_cached_decode():
    """Logits of token T-1 from one prefill of T tokens equal those from a prefill of T-2
    tokens followed by two single-token steps that read the cache."""
    rng = np.random.default_rng(5)
    w, kw = _tiny_weights(rng)
    toks = rng.integers(0, 50, (2, 9))
    full = D.OracleDecoder(w, **kw, batch=2, max_seq=16).forward(toks, 0)
    dec = D.OracleDecoder(w, **kw, batch=2, max_seq=16)
    dec.forward(toks[:, :7], 0)
    dec.forward(toks[:, 7:8], 7)
    last = dec.forward(toks[:, 8:9], 8)
    assert np.allclose(last[:, 0], full[:, -1], rtol=1e-10, atol=1e-10)


def test_generate_feeds_back_the_first_maximum():
    rng = np.random.default_rng(6)
    w, kw = _tiny_weights(rng)
    prompts = rng.integers(0, 50, (2, 4))
    toks, logits = D.OracleDecoder(w, **kw, batch=2, max_seq=16).generate(prompts, 4)
    assert np.array_equal(toks, logits.argmax(axis=-1))
    # the teacher-forced prefill of prompt + generated tokens reproduces the decode logits
    seq = np.concatenate([prompts, toks[:, :-1]], axis=1)
    full = D.OracleDecoder(w, **kw, batch=2, max_seq=16).forward(seq, 0)
    assert np.allclose(full[:, 3:], logits, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("x", [np.array([1.0, 3.0, 3.0, 2.0]), np.array([-np.inf, 0.5, 0.5])])
def test_argmax_convention(x):
    assert int(np.argmax(x)) == int(np.flatnonzero(x == x.max())[0])


def test_silu_is_x_times_the_logistic_function():
    """silu against scipy's logistic function and its known values and limits."""
    from scipy.special import expit

    x = np.linspace(-30, 30, 601)
    assert np.allclose(D.silu(x), x * expit(x), rtol=1e-13, atol=1e-300)
    assert D.silu(np.array([1.0]))[0] == pytest.approx(0.7310585786300049, rel=1e-15)
    assert D.silu(np.array([-1.0]))[0] == pytest.approx(-0.2689414213699951, rel=1e-15)
    assert D.silu(np.array([0.0]))[0] == 0.0
    assert D.silu(np.array([-1000.0]))[0] == 0.0 and D.silu(np.array([50.0]))[0] == pytest.approx(50.0)


def test_swiglu_gates_with_the_even_rows():
    """Row 2i of the gate|up weight is gate i (through silu), row 2i + 1 is up i: with gate rows
    picking x0 and up rows 2 x1, output i is silu(x0) * 2 x1 -- the swapped convention would give
    silu(2 x1) * x0."""
    F, d = 3, 4
    wgu = np.zeros((2 * F, d))
    wgu[0::2, 0] = 1.0
    wgu[1::2, 1] = 2.0
    layer = D.OracleLayer(np.ones(d), np.zeros((1, d)), np.zeros((d, 1)), np.ones(d), wgu, np.zeros((d, F)))
    dec = D.OracleDecoder(D.OracleWeights(np.zeros((1, d)), [layer], np.ones(d), np.zeros((1, d))), 1, 1, d, F,
                          1e-5, 1e4, 1, 4)
    x = np.array([[1.5, -0.75, 3.0, 9.0]])
    got = dec.swiglu(0, x)
    assert np.allclose(got, D.silu(np.array(1.5)) * 2 * -0.75)
    assert not np.allclose(got, D.silu(np.array(2 * -0.75)) * 1.5)
