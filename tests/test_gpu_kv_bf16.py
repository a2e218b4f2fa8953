"""The bf16 KV cache (kv_bytes_per_elem = 2, include/memory_budget.h:37-42) against the
oracle's bf16-cache restatement (orc_attn_core_ex, checked against torch's bf16 cast).

What is exact and what carries a tolerance:
  * history rows a kernel does not write stay bit-identical; an appended V row is the input
    rounded to nearest even, bit for bit;
  * an appended K row is rmsnorm + RoPE of the input, rounded to bf16. The device's fp32 row
    agrees with the oracle's to ~1e-7 relative, so an element within that distance of a bf16
    rounding midpoint may round the other way: K rows are allowed one bf16 ulp on at most
    KEY_FLIP_FRACTION of their elements and must be identical elsewhere (in the whole model
    the V row is a matvec output and gets the same rule);
  * the attention output is checked at the 1e-5 bar against the oracle's attention over the
    very cache contents the kernel left (append off), so the rounding ambiguity above does
    not enter it;
  * whole-model runs compare with the oracle model storing bf16 rows (MODEL_BF16_TOL: one
    flipped row element moves a layer's attention output by up to ~1e-4 relative) and report
    the distance from the fp32-cache model (MODEL_VS_FP32_TOL, the price of the format).
"""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, bf16_bits, bf16_to_f32, golden, rel_l2

pytestmark = pytest.mark.gpu
KEY_FLIP_FRACTION = 2e-3
MODEL_BF16_TOL = 2e-4
MODEL_VS_FP32_TOL = 3e-2


@pytest.fixture(scope="module")
def hip():
    return pyq35.Hip()


class Bufs:
    def __init__(self, hip):
        self.hip, self.p = hip, {}

    def up(self, name, a):
        self.p[name] = self.hip.upload(a)
        return self.p[name]

    def alloc(self, name, nbytes):
        self.p[name] = self.hip.malloc(nbytes)
        return self.p[name]

    def free(self):
        for v in self.p.values():
            self.hip.free(v)
        self.p = {}


def check_key_rows(dev, ref32):
    """dev: bf16 rows read back (fp32); ref32: the oracle's fp32 rows before rounding."""
    want = op.round_bf16(ref32)
    d = dev.view(np.uint32).astype(np.int64) - want.view(np.uint32).astype(np.int64)
    d = d >> 16  # both are bf16 values: count ulps in the top half
    assert np.abs(d).max() <= 1, "appended key off by more than one bf16 ulp"
    frac = np.count_nonzero(d) / d.size
    assert frac <= KEY_FLIP_FRACTION, f"{frac:.3g} of key elements rounded the other way"


def cache_bits(rng, shape, n_filled):
    c = np.zeros(shape, np.float32)
    c[:, :n_filled] = rng.standard_normal(c[:, :n_filled].shape)
    return bf16_bits(c)


def run_attn_decode_bf16(hip, nq, nkv, pos, maxc, n_splits, seed, layers=1):
    rng = np.random.default_rng(seed)
    d = pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)
    HD = 256
    L = layers
    qg = rng.standard_normal((L, 2 * nq * HD)).astype(np.float32)
    kn = rng.standard_normal((L, nkv * HD)).astype(np.float32)
    vn = rng.standard_normal((L, nkv * HD)).astype(np.float32)
    qw = (0.1 * rng.standard_normal((L, HD))).astype(np.float32)
    kw = (0.1 * rng.standard_normal((L, HD))).astype(np.float32)
    Kb = np.stack([cache_bits(rng, (nkv, maxc, HD), pos) for _ in range(L)])  # [L][NKV][ctx][HD]
    Vb = np.stack([cache_bits(rng, (nkv, maxc, HD), pos) for _ in range(L)])
    B = Bufs(hip)
    try:
        args = pyq35.AttnDecodeArgs(q_heads=nq, kv_heads=nkv, head_dim=HD, rotary_dim=64, pos=pos,
                                    n_splits=n_splits, n_layers=L, kv_dtype=1, max_context=maxc,
                                    rope_theta=d.rope_theta, eps=d.rms_norm_eps)
        ws = pyq35.lib.q35_attn_decode_workspace_bytes(args)
        args.qg, args.k_new, args.v_new = B.up("qg", qg), B.up("kn", kn), B.up("vn", vn)
        args.q_norm, args.k_norm = B.up("qw", qw), B.up("kw", kw)
        args.k_cache, args.v_cache = B.up("K", Kb), B.up("V", Vb)
        args.out = B.alloc("out", L * nq * HD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_attn_decode(args, None))
        hip.sync()
        out = hip.download(B.p["out"], (L, nq * HD))
        Kdev = hip.download(B.p["K"], Kb.shape, np.uint16)
        Vdev = hip.download(B.p["V"], Vb.shape, np.uint16)
    finally:
        B.free()
    for l in range(L):
        # history untouched, value row = RNE(v_new) exactly
        np.testing.assert_array_equal(np.delete(Kdev[l], pos, axis=1), np.delete(Kb[l], pos, axis=1))
        np.testing.assert_array_equal(np.delete(Vdev[l], pos, axis=1), np.delete(Vb[l], pos, axis=1))
        np.testing.assert_array_equal(Vdev[l][:, pos], bf16_bits(vn[l]).reshape(nkv, HD))
        # key row vs the oracle's fp32 row, rounded
        K32 = np.ascontiguousarray(bf16_to_f32(Kb[l]).transpose(1, 0, 2))
        V32 = np.ascontiguousarray(bf16_to_f32(Vb[l]).transpose(1, 0, 2))
        op.attn_core_ex(d, pos, qg[l], kn[l], vn[l], qw[l], kw[l], K32, V32, False, True)
        check_key_rows(bf16_to_f32(Kdev[l][:, pos]), K32[pos])
        # output vs the oracle's attention over exactly the cache the kernel left
        Kd = np.ascontiguousarray(bf16_to_f32(Kdev[l]).transpose(1, 0, 2))
        Vd = np.ascontiguousarray(bf16_to_f32(Vdev[l]).transpose(1, 0, 2))
        ref = op.attn_core_ex(d, pos, qg[l], kn[l], vn[l], qw[l], kw[l], Kd, Vd, True, False)
        e = rel_l2(out[l], ref)
        assert e < REL_L2, f"layer {l}: rel_l2 {e}"


@pytest.mark.parametrize("nq,nkv,pos,maxc", [
    (2, 1, 0, 3), (16, 2, 1, 4), (16, 2, 33, 40), (8, 2, 100, 103), (16, 1, 64, 70),
    (16, 2, 2047, 2048),   # the 2B head shape (GQA 8:1) at 2k / 8k
    (16, 2, 8191, 8192),
    (16, 2, 131071, 131072),  # the long-decode context
])
def test_attn_decode_bf16(hip, nq, nkv, pos, maxc):
    run_attn_decode_bf16(hip, nq, nkv, pos, maxc, 0, seed=pos * 7 + nq)


@pytest.mark.parametrize("n_splits", [1, 64])
def test_attn_decode_bf16_split_invariance(hip, n_splits):
    run_attn_decode_bf16(hip, 16, 2, 3000, 4096, n_splits, seed=91)


@pytest.mark.parametrize("pos,n_splits", [(8192, 128), (9200, 128), (9700, 128), (9, 4)])
def test_attn_decode_bf16_split_shapes(hip, pos, n_splits):
    """Splits just past a multiple of the tile, ragged and shorter than a tile, bf16 cache."""
    run_attn_decode_bf16(hip, 16, 2, pos, pos + 1, n_splits, seed=pos + 3)


def test_attn_decode_bf16_layer_batch(hip):
    """Three layers in one launch: each layer's cache starts maxc * NKV * HD bf16 elements on."""
    run_attn_decode_bf16(hip, 8, 2, 700, 800, 0, seed=5, layers=3)


@pytest.mark.parametrize("nq,nkv,T,pos0", [
    (2, 1, 1, 0), (2, 1, 70, 0), (8, 2, 65, 37), (16, 2, 130, 0), (16, 2, 200, 1000),
])
def test_attn_prefill_bf16(hip, nq, nkv, T, pos0):
    rng = np.random.default_rng(T + pos0)
    d = pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)
    HD = 256
    maxc = pos0 + T + 5
    ld = 2 * nq * HD + 2 * nkv * HD
    rows = rng.standard_normal((T, ld)).astype(np.float32)
    qnw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    knw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    Kb = cache_bits(rng, (nkv, maxc, HD), pos0)
    Vb = cache_bits(rng, (nkv, maxc, HD), pos0)
    B = Bufs(hip)
    try:
        args = pyq35.AttnPrefillArgs(n_tokens=T, pos0=pos0, q_heads=nq, kv_heads=nkv, head_dim=HD,
                                     rotary_dim=64, kv_dtype=1, max_context=maxc, rope_theta=d.rope_theta,
                                     eps=d.rms_norm_eps, ld_qkv=ld)
        ws = pyq35.lib.q35_attn_prefill_workspace_bytes(args)
        args.qkv = B.up("rows", rows)
        args.q_norm, args.k_norm = B.up("qn", qnw), B.up("kn", knw)
        args.k_cache, args.v_cache = B.up("K", Kb), B.up("V", Vb)
        args.out = B.alloc("out", T * nq * HD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_attn_prefill(args, None))
        hip.sync()
        out = hip.download(B.p["out"], (T, nq * HD))
        Kdev = hip.download(B.p["K"], Kb.shape, np.uint16)
        Vdev = hip.download(B.p["V"], Vb.shape, np.uint16)
    finally:
        B.free()
    q0, k0, v0 = 0, 2 * nq * HD, 2 * nq * HD + nkv * HD
    np.testing.assert_array_equal(Kdev[:, :pos0], Kb[:, :pos0])
    np.testing.assert_array_equal(Vdev[:, :pos0], Vb[:, :pos0])
    np.testing.assert_array_equal(Vdev[:, pos0:pos0 + T], bf16_bits(rows[:, v0:].reshape(T, nkv, HD)).transpose(1, 0, 2))
    # fp32 key rows from the oracle, one token at a time on a scratch cache
    K32 = np.zeros((maxc, nkv, HD), np.float32)
    V32 = np.zeros_like(K32)
    for t in range(T):
        r = rows[t]
        op.attn_core_ex(d, pos0 + t, r[q0:k0], r[k0:v0], r[v0:], qnw, knw, K32, V32, False, True)
    check_key_rows(bf16_to_f32(Kdev[:, pos0:pos0 + T]).transpose(1, 0, 2), K32[pos0:pos0 + T])
    Kd = np.ascontiguousarray(bf16_to_f32(Kdev).transpose(1, 0, 2))
    Vd = np.ascontiguousarray(bf16_to_f32(Vdev).transpose(1, 0, 2))
    errs = []
    for t in range(T):
        r = rows[t]
        ref = op.attn_core_ex(d, pos0 + t, r[q0:k0], r[k0:v0], r[v0:], qnw, knw, Kd, Vd, True, False)
        errs.append(rel_l2(out[t], ref))
    print(f"worst per-token rel_l2 {max(errs):.3g}")
    assert max(errs) < REL_L2, f"token {int(np.argmax(errs))}: {max(errs)}"


# ----------------------------------------------------------------------------- model level
@pytest.mark.parametrize("name", ["tiny", "tiny_gqa"])
def test_model_bf16_kv_decode_vs_oracle(model_dirs, name):
    g = golden(name)
    prompt = [int(t) for t in g["prompt"]] + [int(t) for t in g["long_ids"][:40]]
    m = pyq35.Model(model_dirs[name], 600, kv_bytes_per_elem=2)
    o = op.Oracle(model_dirs[name], 600, kv_bf16=True)
    otrace = o.enable_trace()
    m.set_layer_trace(True)
    worst, worst32 = 0.0, 0.0
    try:
        for t, tok in enumerate(prompt):
            lg, _ = m.step(tok)
            ref = o.step(tok)
            e = rel_l2(lg, ref)
            tr, otr = m.layer_trace(), otrace[0]
            e = max([e] + [rel_l2(tr[l], otr[l]) for l in range(tr.shape[0])])
            worst = max(worst, e)
            assert e < MODEL_BF16_TOL, f"step {t}: {e}"
            if t < len(g["prompt"]):
                worst32 = max(worst32, rel_l2(lg, g["logits"][t]))
        K, V = m.kv(0, 0, len(prompt))
        # in the model the value row is a matvec output too: both rows carry the midpoint rule
        check_key_rows(K, o.kcache(0)[:len(prompt)])
        check_key_rows(V, o.vcache(0)[:len(prompt)])
    finally:
        m.close()
        o.close()
    print(f"{name}: bf16 cache vs oracle (bf16 rows) worst rel_l2 {worst:.3g}; "
          f"vs the fp32-cache golden logits {worst32:.3g}")
    assert worst32 < MODEL_VS_FP32_TOL


def test_model_bf16_kv_prefill_then_decode(model_dirs):
    """Chunked prefill into a bf16 cache, then decode steps, vs the oracle stepping the same
    ids with bf16 rows."""
    g = golden("tiny")
    ids = [int(t) for t in g["long_ids"][:150]]
    m = pyq35.Model(model_dirs["tiny"], 600, kv_bytes_per_elem=2)
    m.set_prefill_block(64)
    o = op.Oracle(model_dirs["tiny"], 600, kv_bf16=True)
    try:
        lg = m.prefill(ids[:130])
        worst = 0.0
        for t in range(130):
            worst = max(worst, rel_l2(lg[t], o.step(ids[t])))
        for t in range(130, 150):
            l2, _ = m.step(ids[t])
            worst = max(worst, rel_l2(l2, o.step(ids[t])))
    finally:
        m.close()
        o.close()
    print(f"prefill + decode worst logits rel_l2 {worst:.3g}")
    assert worst < MODEL_BF16_TOL


def test_model_bf16_kv_arena_and_io(model_dirs):
    """Half the KV bytes; host writes are rounded to nearest even and read back exactly;
    fill_synthetic writes bf16 values of unit spread."""
    m32 = pyq35.Model(model_dirs["tiny"], 1024)
    m16 = pyq35.Model(model_dirs["tiny"], 1024, kv_bytes_per_elem=2)
    try:
        assert m16.budget()["kv_cache_bytes"] * 2 == m32.budget()["kv_cache_bytes"]
        d = m16.dims
        rng = np.random.default_rng(3)
        k = rng.standard_normal((50, d.attn_kv_heads, d.attn_head_dim)).astype(np.float32)
        v = rng.standard_normal(k.shape).astype(np.float32)
        m16.set_kv(0, 900, k, v)
        K, V = m16.kv(0, 900, 50)
        np.testing.assert_array_equal(K, op.round_bf16(k))
        np.testing.assert_array_equal(V, op.round_bf16(v))
        m16.fill_synthetic(800, seed=11, state_std=0.1)
        m32.fill_synthetic(800, seed=11, state_std=0.1)
        K16, V16 = m16.kv(0, 0, 800)
        K32, V32 = m32.kv(0, 0, 800)
        np.testing.assert_array_equal(K16, op.round_bf16(K32))
        np.testing.assert_array_equal(V16, op.round_bf16(V32))
        m16.step(1)
        assert m16.position == 801
    finally:
        m16.close()
        m32.close()
