"""Closed-form and brute-force checks of the oracle's primitives and mixers: properties the
mathematics fixes, chosen so that a dropped term, a wrong sign or index or a transposed
operand fails one of them (the golden vectors pin the same functions against the
reference engine)."""
import math

import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import bf16_bits, bf16_to_f32, rel_l2

rng = np.random.default_rng(1234)
D = pyq35.dims_for("tiny")  # GDN 2 k/v heads of 128, attention 2 q / 1 kv heads of 256


def test_bf16_widening_and_matvec_exact():
    # weights and inputs that are exact in bf16/fp32 with exact fp32 products and sums
    W = rng.integers(-8, 9, size=(37, 96)).astype(np.float32) * 0.25
    x = rng.integers(-16, 17, size=96).astype(np.float32)
    Wb = bf16_bits(W)
    np.testing.assert_array_equal(bf16_to_f32(Wb), W)
    y = op.matmul_bf16(Wb, x)
    np.testing.assert_array_equal(y, (W.astype(np.float64) @ x).astype(np.float32))


def test_matvec_brute_force():
    for rows, cols in [(5, 8), (17, 40), (64, 1000), (3, 2051)]:
        W = bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32))
        x = rng.standard_normal(cols).astype(np.float32)
        ref = bf16_to_f32(W).astype(np.float64) @ x.astype(np.float64)
        y = op.matmul_bf16(W, x)
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.sqrt(cols) * np.max(np.abs(ref))


def test_rmsnorm_closed_form():
    eps = 1e-6
    x = rng.standard_normal(1024).astype(np.float32) * 3
    ms = float(np.mean(x.astype(np.float64) ** 2))
    y = op.rmsnorm(x, np.zeros(1024, np.float32), eps)
    assert abs(np.mean(y.astype(np.float64) ** 2) - ms / (ms + eps)) < 1e-6
    # (1 + w) form: w = 1 doubles the output; a per-element weight scales that element
    y2 = op.rmsnorm(x, np.ones(1024, np.float32), eps)
    np.testing.assert_allclose(y2, 2 * y, rtol=1e-6)
    w = np.zeros(1024, np.float32)
    w[7] = 2.0
    y3 = op.rmsnorm(x, w, eps)
    assert abs(y3[7] - 3 * y[7]) <= 1e-6 * abs(y[7]) + 1e-12
    np.testing.assert_array_equal(np.delete(y3, 7), np.delete(y, 7))


def test_l2norm_closed_form():
    eps = 1e-6
    for scale in (1e-3, 1.0, 30.0):
        x = rng.standard_normal(128).astype(np.float32) * scale
        s = float(np.sum(x.astype(np.float64) ** 2))
        y = op.l2norm(x, eps)
        assert abs(np.sum(y.astype(np.float64) ** 2) - s / (s + eps)) < 1e-6
        np.testing.assert_allclose(y / np.linalg.norm(y), x / np.linalg.norm(x), rtol=1e-5, atol=1e-7)


def test_rmsnorm_gated_limits():
    eps = 1e-6
    x = rng.standard_normal(128).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    base = op.rmsnorm(x, w - 1.0, eps)  # w * x * rsqrt(...)
    y0 = op.rmsnorm_gated(x, w, np.zeros(128, np.float32), eps)
    np.testing.assert_array_equal(y0, np.zeros(128, np.float32))
    z = np.full(128, 60.0, np.float32)  # silu(60) == 60 in fp32
    y = op.rmsnorm_gated(x, w, z, eps)
    np.testing.assert_allclose(y, base * 60.0, rtol=2e-6)


def test_rope_properties():
    theta, rot, hd = 1e7, 64, 256
    x = rng.standard_normal(hd).astype(np.float32)
    np.testing.assert_array_equal(op.apply_rope(x, rot, 0, theta), x)
    for pos in (1, 17, 8191, 131071):
        y = op.apply_rope(x, rot, pos, theta)
        np.testing.assert_array_equal(y[rot:], x[rot:])
        h = rot // 2
        for i in range(h):  # each (i, i+h) pair is rotated by pos * theta^(-2i/rot)
            assert abs(math.hypot(y[i], y[i + h]) - math.hypot(x[i], x[i + h])) < 1e-5
        ang = pos * theta ** (-np.arange(h, dtype=np.float64) * 2 / rot)
        c, s = np.cos(ang), np.sin(ang)
        ref_lo = x[:h] * c - x[h:rot] * s
        ref_hi = x[h:rot] * c + x[:h] * s
        np.testing.assert_allclose(y[:h], ref_lo, atol=2e-6)
        np.testing.assert_allclose(y[h:rot], ref_hi, atol=2e-6)


# ----------------------------------------------------------------------------- GDN core
CONV = 2 * D.gdn_k_heads * 128 + D.gdn_v_heads * 128
KD = D.gdn_k_heads * 128
VD = D.gdn_v_heads * 128


def _gdn_inputs(qkv=None, b=0.0, a=0.0, A_log=0.0, taps=(0, 0, 0, 1)):
    qkv = rng.standard_normal(CONV).astype(np.float32) if qkv is None else qkv
    conv_w = np.tile(np.asarray(taps, np.float32), CONV)
    return dict(qkv=qkv, z=np.ones(VD, np.float32), b=np.full(D.gdn_v_heads, b, np.float32),
                a=np.full(D.gdn_v_heads, a, np.float32), conv_w=conv_w,
                A_log=np.full(D.gdn_v_heads, A_log, np.float32),
                dt_bias=np.zeros(D.gdn_v_heads, np.float32), norm_w=np.ones(128, np.float32))


def _silu(x):
    x = x.astype(np.float64)
    return x / (1 + np.exp(-x))


def test_conv_window_shift_and_impulse():
    win = np.zeros((CONV, 3), np.float32)
    S = np.zeros((D.gdn_v_heads, 128, 128), np.float32)
    taps = (0.5, -0.25, 2.0, 1.0)
    xs = [rng.standard_normal(CONV).astype(np.float32) for _ in range(4)]
    for t, x in enumerate(xs):
        op.gdn_core(D, **_gdn_inputs(qkv=x, taps=taps), conv_win=win, S=S)
        # the window holds the last three inputs, oldest first (zeros before t = 0)
        for k in range(3):
            src = t - 2 + k
            np.testing.assert_array_equal(win[:, k], xs[src] if src >= 0 else 0.0)


def test_conv_impulse_response():
    """A unit input on every channel at t = 0, then zeros: the v readout of step t carries
    silu(tap[3 - t]) -- the taps newest-first. k channels get a constant input so that
    k is a fixed unit vector; beta = 1, alpha = 1 and S = 0 make S' = k v^T and the
    readout v (k . q) with q = k / sqrt(DK)."""
    taps = (0.5, -0.25, 2.0, 1.0)
    win = np.zeros((CONV, 3), np.float32)
    for t in range(4):
        x = np.zeros(CONV, np.float32)
        x[KD:] = 1.0 if t == 0 else 0.0
        S = np.zeros((D.gdn_v_heads, 128, 128), np.float32)
        # k channels: keep their conv output constant by refreshing the window each step
        win[KD:2 * KD] = 0.0
        x[KD:2 * KD] = 1.0
        x[:KD] = 1.0
        win[:KD] = 0.0
        raw, _ = op.gdn_core(D, **_gdn_inputs(qkv=x, b=40.0, A_log=-100.0, taps=taps), conv_win=win, S=S)
        k = np.full(128, 1 / math.sqrt(128 + 1e-6 / _silu(np.array([1.0]))[0] ** 2))
        kq = float(k @ k) / math.sqrt(128)
        expect = _silu(np.array([taps[3 - t]]))[0] * kq
        np.testing.assert_allclose(raw, expect, rtol=1e-5)


def test_delta_rule_fixed_point():
    """beta = 1, alpha = 1: after one update S^T k == v (|k| = 1); with q's conv inputs equal
    to k's, the readout is v / sqrt(DK) scaled by |k|^2."""
    x = rng.standard_normal(CONV).astype(np.float32)
    x[:KD] = x[KD:2 * KD]  # q channels = k channels
    S = (0.1 * rng.standard_normal((D.gdn_v_heads, 128, 128))).astype(np.float32)
    win = np.zeros((CONV, 3), np.float32)
    raw, _ = op.gdn_core(D, **_gdn_inputs(qkv=x, b=40.0, A_log=-100.0), conv_win=win, S=S)
    v = _silu(x[2 * KD:]).reshape(D.gdn_v_heads, 128)
    for h in range(D.gdn_v_heads):
        kc = _silu(x[KD + h * 128:KD + (h + 1) * 128])
        s = float(np.sum(kc ** 2))
        k = kc / math.sqrt(s + 1e-6)
        kk = float(k @ k)
        # S'^T k = S^T k (1 - kk) + v kk
        assert np.max(np.abs(S[h].T.astype(np.float64) @ k - v[h])) < 1e-4
        np.testing.assert_allclose(raw[h * 128:(h + 1) * 128], v[h] * kk / math.sqrt(128),
                                   rtol=1e-4, atol=1e-5)


def _silu_inverse(y):
    """x > 0 with x / (1 + e^-x) = y (y > 0), by bisection in float64."""
    lo, hi = np.zeros_like(y), np.maximum(2.0 * y + 2.0, 1.0)
    for _ in range(80):
        mid = 0.5 * (lo + hi)
        big = _silu(mid) > y
        hi = np.where(big, mid, hi)
        lo = np.where(big, lo, mid)
    return 0.5 * (lo + hi)


def test_delta_rule_linear_in_v():
    """From S = 0, with q, k, beta, alpha fixed, the delta rule is linear in v:
    S_t = alpha S_{t-1} + beta k (v_t - S_{t-1}^T k)^T, so doubling every v doubles every S_t
    and every readout S_t^T q. v reaches the rule as silu(conv(x_v)); with taps passing the
    current input through, the v inputs of the doubled run are silu^-1(2 silu(x_v)), and
    the fp32 values that reach the rule differ from 2 v by a few ulp."""
    seq = [rng.standard_normal(CONV).astype(np.float32) for _ in range(6)]
    for x in seq:
        x[2 * KD:] = np.abs(x[2 * KD:]) + 0.25  # v inputs > 0: silu is invertible there
    runs = []
    for double in (False, True):
        S = np.zeros((D.gdn_v_heads, 128, 128), np.float32)
        win = np.zeros((CONV, 3), np.float32)
        outs = []
        for x in seq:
            xx = x.copy()
            if double:
                xx[2 * KD:] = _silu_inverse(2.0 * _silu(x[2 * KD:])).astype(np.float32)
            raw, _ = op.gdn_core(D, **_gdn_inputs(qkv=xx, b=0.1, a=0.2, A_log=0.0), conv_win=win, S=S)
            outs.append(raw)
        runs.append((S.copy(), np.stack(outs)))
    (S1, o1), (S2, o2) = runs
    assert np.abs(S1).max() > 0.1  # the state is not trivially zero
    assert rel_l2(S2, 2.0 * S1) < 2e-6
    assert rel_l2(o2, 2.0 * o1) < 2e-6
    # a v that does not scale (the same input) is not mistaken for linear behaviour
    assert rel_l2(S1, 2.0 * S1) > 0.4


def test_decay_reset():
    """alpha -> 0 erases the state: S' = beta k v^T."""
    x = rng.standard_normal(CONV).astype(np.float32)
    S = (rng.standard_normal((D.gdn_v_heads, 128, 128))).astype(np.float32)
    win = np.zeros((CONV, 3), np.float32)
    op.gdn_core(D, **_gdn_inputs(qkv=x, b=0.3, a=30.0, A_log=10.0), conv_win=win, S=S)
    beta = 1 / (1 + math.exp(-0.3))
    for h in range(D.gdn_v_heads):
        kc = _silu(x[KD + h * 128:KD + (h + 1) * 128])
        k = kc / math.sqrt(float(np.sum(kc ** 2)) + 1e-6)
        v = _silu(x[2 * KD + h * 128:2 * KD + (h + 1) * 128])
        np.testing.assert_allclose(S[h], beta * np.outer(k, v), rtol=2e-5, atol=1e-7)


def test_gdn_core_brute_force_float64():
    """A float64 restatement of one token (conv, l2norm, decay, delta rule, readout, gated
    norm) on random inputs."""
    x = rng.standard_normal(CONV).astype(np.float32)
    win = rng.standard_normal((CONV, 3)).astype(np.float32)
    S = (0.1 * rng.standard_normal((D.gdn_v_heads, 128, 128))).astype(np.float32)
    inp = _gdn_inputs(qkv=x, b=0.4, a=-0.7, A_log=0.3, taps=(0.3, -0.2, 0.1, 0.9))
    inp["z"] = rng.standard_normal(VD).astype(np.float32)
    inp["norm_w"] = rng.standard_normal(128).astype(np.float32)
    S64 = S.astype(np.float64).copy()
    w64 = win.astype(np.float64)
    taps = np.array([0.3, -0.2, 0.1, 0.9])
    conv = _silu((w64 * taps[:3]).sum(axis=1) + taps[3] * x)
    raw, out = op.gdn_core(D, **inp, conv_win=win, S=S)
    g = -math.exp(0.3) * math.log1p(math.exp(-0.7))
    alpha, beta = math.exp(g), 1 / (1 + math.exp(-0.4))
    for h in range(D.gdn_v_heads):
        q = conv[h * 128:(h + 1) * 128]
        k = conv[KD + h * 128:KD + (h + 1) * 128]
        v = conv[2 * KD + h * 128:2 * KD + (h + 1) * 128]
        q = q / math.sqrt(np.sum(q * q) + 1e-6) / math.sqrt(128)
        k = k / math.sqrt(np.sum(k * k) + 1e-6)
        Sh = alpha * S64[h]
        Sh = Sh + np.outer(k, (v - Sh.T @ k) * beta)
        o = Sh.T @ q
        np.testing.assert_allclose(S[h], Sh, rtol=1e-4, atol=2e-6)
        np.testing.assert_allclose(raw[h * 128:(h + 1) * 128], o, rtol=1e-4, atol=2e-6)
        ms = np.mean(o * o)
        zz = inp["z"][h * 128:(h + 1) * 128].astype(np.float64)
        ref = inp["norm_w"] * (o / np.sqrt(ms + D.rms_norm_eps)) * zz / (1 + np.exp(-zz))
        np.testing.assert_allclose(out[h * 128:(h + 1) * 128], ref, rtol=1e-4, atol=1e-6)


# ----------------------------------------------------------------------------- attention
def _attn_case(pos, same_keys=False):
    NQ, NKV = D.attn_q_heads, D.attn_kv_heads
    qg = rng.standard_normal(2 * NQ * 256).astype(np.float32)
    kn = rng.standard_normal(NKV * 256).astype(np.float32)
    vn = rng.standard_normal(NKV * 256).astype(np.float32)
    K = np.zeros((pos + 1, NKV, 256), np.float32)
    V = np.zeros_like(K)
    K[:pos] = rng.standard_normal((pos, NKV, 256))
    V[:pos] = rng.standard_normal((pos, NKV, 256))
    return qg, kn, vn, K, V


def test_attention_first_position_is_gated_value():
    qg, kn, vn, K, V = _attn_case(0)
    w0 = np.zeros(256, np.float32)
    out = op.attn_core(D, 0, qg, kn, vn, w0, w0, K, V)
    gate = qg.reshape(D.attn_q_heads, 2, 256)[:, 1]
    ref = vn.reshape(D.attn_kv_heads, 256)[np.arange(D.attn_q_heads) // (D.attn_q_heads // D.attn_kv_heads)]
    np.testing.assert_allclose(out.reshape(D.attn_q_heads, 256), ref / (1 + np.exp(-gate.astype(np.float64))),
                               rtol=1e-6)


def test_attention_brute_force_float64():
    pos = 40
    qg, kn, vn, K, V = _attn_case(pos)
    qn = rng.standard_normal(256).astype(np.float32) * 0.1
    knw = rng.standard_normal(256).astype(np.float32) * 0.1
    out = op.attn_core(D, pos, qg, kn, vn, qn, knw, K, V)
    NQ, NKV = D.attn_q_heads, D.attn_kv_heads
    grp = NQ // NKV
    # the appended key is normed + rotated, the value is copied
    for kh in range(NKV):
        kref = op.apply_rope(op.rmsnorm(kn[kh * 256:(kh + 1) * 256], knw, D.rms_norm_eps), 64, pos, D.rope_theta)
        np.testing.assert_array_equal(K[pos, kh], kref)
    np.testing.assert_array_equal(V[pos], vn.reshape(NKV, 256))
    for h in range(NQ):
        q = op.apply_rope(op.rmsnorm(qg[h * 512:h * 512 + 256], qn, D.rms_norm_eps), 64, pos, D.rope_theta)
        kh = h // grp
        s = (K[:pos + 1, kh].astype(np.float64) @ q.astype(np.float64)) / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        o = p @ V[:pos + 1, kh].astype(np.float64)
        gate = qg[h * 512 + 256:(h + 1) * 512].astype(np.float64)
        np.testing.assert_allclose(out[h * 256:(h + 1) * 256], o / (1 + np.exp(-gate)), rtol=2e-5, atol=1e-6)


def test_attention_identical_keys_average_values():
    pos = 20
    qg, kn, vn, K, V = _attn_case(pos)
    w0 = np.zeros(256, np.float32)
    # make every cached key equal to the new (normed + rotated) key: uniform weights
    kk = op.apply_rope(op.rmsnorm(kn[:256], w0, D.rms_norm_eps), 64, pos, D.rope_theta)
    K[:pos, 0] = kk
    out = op.attn_core(D, pos, qg, kn, vn, w0, w0, K, V)
    gate = qg.reshape(D.attn_q_heads, 2, 256)[:, 1].astype(np.float64)
    mean_v = V[:pos + 1, 0].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(out.reshape(D.attn_q_heads, 256), mean_v / (1 + np.exp(-gate)),
                               rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("x", [-30.0, -1.0, 0.0, 0.5, 19.9, 20.0, 20.1, 80.0])
def test_scalar_activations(x):
    assert op.olib.orc_softplus(x) == pytest.approx(x if x > 20 else math.log1p(math.exp(x)), rel=1e-6)
    assert op.olib.orc_sigmoid(x) == pytest.approx(1 / (1 + math.exp(-x)), rel=1e-6, abs=1e-30)
    assert op.olib.orc_silu(x) == pytest.approx(x / (1 + math.exp(-x)), rel=1e-6, abs=1e-30)


def test_round_bf16_matches_torch_cast():
    """The bf16 cache rounding against torch's fp32 -> bfloat16 cast (nearest, ties to even):
    random values, exact ties both ways, subnormals, the overflow edge, infinities, NaN."""
    torch = pytest.importorskip("torch")
    base = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000)
    hi = (rng.integers(0, 1 << 16, 4000, dtype=np.uint32) << 16)
    ties = np.concatenate([hi | 0x8000, (hi | 0x18000) & 0xffffffff, hi | 0x7fff, hi | 0x8001]).view(np.float32)
    special = np.array([0.0, -0.0, 1e-45, -1e-45, 1e-40, 3.389e38, 3.4e38, -3.4e38, np.inf, -np.inf,
                        3.4028235e38, 1.1754944e-38], np.float32)
    x = np.concatenate([base, ties[np.isfinite(ties)], special]).astype(np.float32)
    got = op.round_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(op.olib.orc_round_bf16(float("nan")))
    # every result is a bf16 value and the nearest one
    assert not np.any(got[np.isfinite(got)].view(np.uint32) & 0xffff)
    assert op.round_bf16(np.float32(1.00390625)) == 1.0        # tie (1 + 2^-8) -> even 1.0
    assert op.round_bf16(np.float32(1.01171875)) == 1.015625   # tie (1 + 3 * 2^-8) -> even


def test_attention_bf16_cache_rounds_appended_rows():
    """kv_bf16: the appended rows are the fp32 rows rounded to bf16 and the output equals the
    attention over the rounded caches (append off on the same contents); with bf16-exact
    history the fp32 and bf16 paths differ only through the rounded row."""
    pos = 33
    qg, kn, vn, K, V = _attn_case(pos)
    K[:pos] = op.round_bf16(K[:pos])
    V[:pos] = op.round_bf16(V[:pos])
    qn = rng.standard_normal(256).astype(np.float32) * 0.1
    knw = rng.standard_normal(256).astype(np.float32) * 0.1
    K32, V32 = K.copy(), V.copy()
    out32 = op.attn_core_ex(D, pos, qg, kn, vn, qn, knw, K32, V32, False, True)
    np.testing.assert_array_equal(out32, op.attn_core(D, pos, qg, kn, vn, qn, knw, K.copy(), V.copy()))
    Kb, Vb = K.copy(), V.copy()
    outb = op.attn_core_ex(D, pos, qg, kn, vn, qn, knw, Kb, Vb, True, True)
    torch = pytest.importorskip("torch")
    as_bf16 = lambda a: torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(Kb[pos], as_bf16(K32[pos]))
    np.testing.assert_array_equal(Vb[pos], as_bf16(V32[pos]))
    np.testing.assert_array_equal(Kb[:pos], K[:pos])
    # the same caches with append off give the same output bit for bit
    zero = np.zeros_like(kn)
    again = op.attn_core_ex(D, pos, qg, zero, zero, qn, knw, Kb.copy(), Vb.copy(), True, False)
    np.testing.assert_array_equal(again, outb)
    # and the output moved by no more than bf16 rounding of one row can move it
    assert 0 < np.linalg.norm(outb - out32) / np.linalg.norm(out32) < 4e-3
