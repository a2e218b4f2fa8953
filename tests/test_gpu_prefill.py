"""The whole-prompt path on the GPU: the token-batched MFMA GEMM (q35_gemm_bf16), the chunked
GDN prefill (q35_gdn_prefill) and the flash attention prefill (q35_attn_prefill) through the
kernel-level C ABI against the oracle's sequential recurrences on the same seeded inputs, and
the model-level prefill (q35_model_prefill / q35_model_extend) against the golden vectors of
the compiled reference (QwenForward::prefill and QwenModel::step logits, per-layer hidden
states) and against token-serial decoding (state handed to decode)."""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, bf16_bits, bf16_to_f32, golden, rel_l2, ring_from_window, window_from_ring

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return pyq35.Hip()


class Bufs:
    def __init__(self, hip):
        self.hip, self.p = hip, {}

    def up(self, name, a):
        self.p[name] = self.hip.upload(np.ascontiguousarray(a))
        return self.p[name]

    def alloc(self, name, nbytes):
        self.p[name] = self.hip.malloc(nbytes)
        return self.p[name]

    def free(self):
        for v in self.p.values():
            self.hip.free(v)
        self.p = {}


# ----------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K,ldx,resid", [
    (1, 8, 32, 32, False), (130, 70, 64, 68, True), (257, 300, 520, 520, False),
    (64, 129, 8, 8, True), (512, 2048, 2048, 2048, True), (1000, 8224, 1024, 1024, False),
    (300, 12290, 136, 136, True), (129, 12288, 64, 72, False),
    (70, 96, 1000, 1000, True), (33, 40, 4104, 4104, False)])  # K past one block of 512 (ragged)
def test_gemm_bf16(hip, M, N, K, ldx, resid):
    rng = np.random.default_rng(M * 7 + N + K)
    X = rng.standard_normal((M, ldx)).astype(np.float32)
    W = bf16_bits(0.02 * rng.standard_normal((N, K)).astype(np.float32))
    R = rng.standard_normal((M, N)).astype(np.float32) if resid else None
    B = Bufs(hip)
    try:
        dX, dW = B.up("X", X), B.up("W", W)
        dY = B.up("Y", R) if resid else B.alloc("Y", M * N * 4)
        pyq35.check(pyq35.lib.q35_gemm_bf16(dX, ldx, dW, M, N, K, dY if resid else None, N, dY, N, None))
        hip.sync()
        Y = hip.download(dY, (M, N))
    finally:
        B.free()
    ref = X[:, :K].astype(np.float64) @ bf16_to_f32(W).astype(np.float64).T
    if resid:
        ref += R
    assert rel_l2(Y, ref) < 1e-6
    np.testing.assert_allclose(Y, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144)])
def test_gemm_accuracy_at_projection_depth(hip, N, K):
    """At the 2B projections' depths the GEMM stays as close to float64 as the matvec does
    (about 1.2e-7 - 1.9e-7): products accumulated in blocks of K = 512 then summed. One fp32
    accumulator over all of K measures 4.9e-7 (K = 2048) and 8.7e-7 (K = 6144) here."""
    M = 256
    rng = np.random.default_rng(N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = bf16_bits(0.02 * rng.standard_normal((N, K)).astype(np.float32))
    B = Bufs(hip)
    try:
        dX, dW, dY = B.up("X", X), B.up("W", W), B.alloc("Y", M * N * 4)
        pyq35.check(pyq35.lib.q35_gemm_bf16(dX, K, dW, M, N, K, None, N, dY, N, None))
        hip.sync()
        Y = hip.download(dY, (M, N))
    finally:
        B.free()
    ref = X.astype(np.float64) @ bf16_to_f32(W).astype(np.float64).T
    err = rel_l2(Y, ref)
    print(f"N={N} K={K}: rel_l2 vs float64 {err:.3g}")
    assert err < 3.5e-7


def test_gemm_rejects_bad_shapes(hip):
    unsupported, bad_arg = -7, -1
    assert pyq35.lib.q35_gemm_bf16(256, 12, 256, 4, 4, 12, None, 4, 512, 4, None) == unsupported  # K % 8
    assert pyq35.lib.q35_gemm_bf16(None, 32, 256, 4, 4, 32, None, 4, 512, 4, None) == bad_arg
    ws = pyq35.lib.q35_gemm_f16x2_workspace_bytes(4, 4, 32)
    assert ws > 0 and pyq35.lib.q35_gemm_f16x2_workspace_bytes(4, 4, 0) == 0
    assert pyq35.lib.q35_gemm_f16x2(256, 40, 256, 4, 4, 40, None, 4, 512, 4, 1 << 20, 1 << 20, None) == unsupported
    assert pyq35.lib.q35_gemm_f16x2(256, 32, 256, 4, 4, 32, None, 4, 512, 4, (1 << 20) + 16, ws, None) == unsupported
    assert pyq35.lib.q35_gemm_f16x2(256, 32, 256, 4, 4, 32, None, 4, 512, 4, 1 << 20, ws - 4, None) == bad_arg


def _f16x2_inputs(M, N, K, seed):
    """Activations with the rows the two-part split has to survive -- all zeros, one channel
    10^4 times the rest, magnitudes near 1e-20 and 1e20 -- and bf16 weights whose
    magnitudes spread log-uniformly down to 2^-30 of the largest."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K)).astype(np.float32)
    X[0] = 0.0
    X[1] = 1e-4 * X[1]
    X[1, K // 3] = 1.0
    X[2] *= np.float32(1e-20)
    X[3] *= np.float32(1e20)
    X[4, : K // 2] = 0.0
    w = 0.02 * rng.standard_normal((N, K)) * np.exp2(-rng.uniform(0, 30, (N, K)))
    w[0, 0] = 0.08  # the largest
    return X, bf16_bits(w.astype(np.float32))


@pytest.mark.parametrize("N,K,resid", [(8224, 2048, False), (2048, 2048, True), (12288, 2048, False),
                                       (2048, 6144, True), (9216, 2048, False), (2048, 4096, True)])
def test_gemm_f16x2_vs_float64(hip, N, K, resid):
    """The model prefill's projection GEMM (two fp16 parts per activation against the scaled
    fp16 weight copy) at the 2B projection shapes against float64, elementwise within
    2^-17 of sum |x||w| (the split's 2^-22 |x| plus fp32 accumulation over K, with headroom)
    and within 1e-6 rel_l2 per ordinary row; zero rows give exact zeros; the three-part
    bf16 path agrees to the same 1e-6."""
    M = 203
    X, W = _f16x2_inputs(M, N, K, N + K)
    R = np.random.default_rng(K).standard_normal((M, N)).astype(np.float32) if resid else None
    ws = pyq35.lib.q35_gemm_f16x2_workspace_bytes(M, N, K)
    B = Bufs(hip)
    try:
        dX, dW, dws = B.up("X", X), B.up("W", W), B.alloc("ws", ws)
        dY = B.up("Y", R) if resid else B.alloc("Y", M * N * 4)
        pyq35.check(pyq35.lib.q35_gemm_f16x2(dX, K, dW, M, N, K, dY if resid else None, N, dY, N, dws, ws, None))
        hip.sync()
        Y = hip.download(dY, (M, N))
        dY3 = B.up("Y3", R) if resid else B.alloc("Y3", M * N * 4)
        pyq35.check(pyq35.lib.q35_gemm_bf16(dX, K, dW, M, N, K, dY3 if resid else None, N, dY3, N, None))
        hip.sync()
        Y3 = hip.download(dY3, (M, N))
    finally:
        B.free()
    Wf = bf16_to_f32(W).astype(np.float64)
    ref = X.astype(np.float64) @ Wf.T
    scale = np.abs(X.astype(np.float64)) @ np.abs(Wf).T
    if resid:
        ref += R
        scale += np.abs(R)
    bound = 2.0**-17 * scale
    worst = float(np.max(np.abs(Y - ref) / np.where(scale > 0, scale, 1.0)))
    print(f"N={N} K={K}: worst |dy| / sum|x||w| = {worst:.3g} (2^{np.log2(max(worst, 1e-300)):.1f})")
    assert np.all(np.abs(Y - ref) <= bound)
    if not resid:
        assert np.all(Y[0] == 0.0)
    for r in range(M):
        if np.abs(ref[r]).max() > 0:
            assert rel_l2(Y[r], ref[r]) < 1e-6, r
            assert rel_l2(Y[r], Y3[r]) < 1e-6, r
    print(f"  rel_l2 vs float64: rows 1-3 {[f'{rel_l2(Y[r], ref[r]):.2g}' for r in (1, 2, 3)]}, "
          f"all {rel_l2(Y, ref):.3g}; vs three-part {rel_l2(Y, Y3):.3g}")


# ----------------------------------------------------------------------------- GDN
def run_gdn_prefill(hip, kh, vh, T, pos0, fused, seed):
    """Chunked prefill of T tokens after pos0 earlier ones vs T sequential oracle steps."""
    rng = np.random.default_rng(seed)
    d = pyq35.default_dims(gdn_k_heads=kh, gdn_v_heads=vh)
    KD, VD = kh * 128, vh * 128
    CONV = 2 * KD + VD
    ld = CONV + VD + 2 * vh + 4  # token rows as the fused in-projection lays them out (+ pad)
    rows = rng.standard_normal((T, ld)).astype(np.float32)
    conv_w = (0.5 * rng.standard_normal(CONV * 4)).astype(np.float32)
    A_log = rng.standard_normal(vh).astype(np.float32)
    dt_bias = rng.standard_normal(vh).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    if pos0 > 0:
        S = (0.1 * rng.standard_normal((vh, 128, 128))).astype(np.float32)
        win = rng.standard_normal((CONV, 3)).astype(np.float32)
    else:
        S = np.zeros((vh, 128, 128), np.float32)
        win = np.zeros((CONV, 3), np.float32)
    B = Bufs(hip)
    try:
        args = pyq35.GdnPrefillArgs(n_tokens=T, pos0=pos0, k_heads=kh, v_heads=vh, head_dim_k=128,
                                    head_dim_v=128, conv_kernel=4, eps=d.rms_norm_eps)
        ws = pyq35.lib.q35_gdn_prefill_workspace_bytes(args)
        base = B.up("rows", rows)
        args.qkv, args.z = base, base + CONV * 4
        args.b, args.a = base + (CONV + VD) * 4, base + (CONV + VD + vh) * 4
        args.ld_qkv = args.ld_z = args.ld_ba = ld
        args.conv_w, args.A_log, args.dt_bias = B.up("cw", conv_w), B.up("al", A_log), B.up("dt", dt_bias)
        args.norm_w = B.up("nw", norm_w) if fused else None
        args.conv_ring = B.up("ring", ring_from_window(win, pos0))
        args.state = B.up("S", S)
        args.out = B.alloc("out", T * VD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_gdn_prefill(args, None))
        hip.sync()
        out = hip.download(B.p["out"], (T, VD))
        S_dev = hip.download(B.p["S"], S.shape)
        ring = hip.download(B.p["ring"], (4, CONV))
    finally:
        B.free()
    S_o, win_o = S.copy(), win.copy()
    ref = np.zeros((T, VD), np.float32)
    for t in range(T):
        r = rows[t]
        raw, normed = op.gdn_core(d, r[:CONV], r[CONV:CONV + VD], r[CONV + VD:CONV + VD + vh],
                                  r[CONV + VD + vh:CONV + VD + 2 * vh], conv_w, A_log, dt_bias, norm_w,
                                  win_o, S_o)
        ref[t] = normed if fused else raw
    return out, ref, S_dev, S_o, window_from_ring(ring, pos0 + T), win_o


@pytest.mark.parametrize("kh,vh,T,pos0,fused", [
    (2, 2, 1, 0, True), (2, 2, 3, 0, False), (2, 2, 63, 0, True), (2, 2, 64, 0, False),
    (2, 2, 65, 5, True), (2, 2, 200, 2, False),
    (2, 2, 1, 5, True), (2, 2, 2, 9, False),  # blocks shorter than the conv window after a ring
    (8, 16, 130, 3, True),      # v-heads = 2 k-heads
    (16, 16, 300, 7, True),     # the 2B / isolated-GDN head shape, ragged last chunk
])
def test_gdn_prefill_vs_sequential(hip, kh, vh, T, pos0, fused):
    out, ref, S_dev, S_o, win, win_o = run_gdn_prefill(hip, kh, vh, T, pos0, fused, seed=T * 13 + kh + pos0)
    errs = [rel_l2(out[t], ref[t]) for t in range(T)]
    print(f"worst per-token rel_l2 {max(errs):.3g}, state rel_l2 {rel_l2(S_dev, S_o):.3g}")
    assert max(errs) < REL_L2, f"token {int(np.argmax(errs))}: {max(errs)}"
    assert rel_l2(S_dev, S_o) < REL_L2
    np.testing.assert_array_equal(win, win_o)


def test_gdn_prefill_512_tokens_state(hip):
    """State after 512 tokens (the decode bar: rel_l2 <= 1e-5 after 512 steps), 16 heads."""
    out, ref, S_dev, S_o, win, win_o = run_gdn_prefill(hip, 16, 16, 512, 0, False, seed=512)
    assert rel_l2(S_dev, S_o) < REL_L2
    assert max(rel_l2(out[t], ref[t]) for t in range(512)) < REL_L2


# ----------------------------------------------------------------------------- attention
def run_attn_prefill(hip, nq, nkv, T, pos0, seed, rot=64, ws_min=False):
    rng = np.random.default_rng(seed)
    d = pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)
    d.partial_rotary_factor = rot / 256.0
    HD = 256
    maxc = pos0 + T + 5
    ld = 2 * nq * HD + 2 * nkv * HD
    rows = rng.standard_normal((T, ld)).astype(np.float32)
    qnw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    knw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    Kd = np.zeros((nkv, maxc, HD), np.float32)
    Vd = np.zeros_like(Kd)
    Kd[:, :pos0] = rng.standard_normal((nkv, pos0, HD))
    Vd[:, :pos0] = rng.standard_normal((nkv, pos0, HD))
    B = Bufs(hip)
    try:
        args = pyq35.AttnPrefillArgs(n_tokens=T, pos0=pos0, q_heads=nq, kv_heads=nkv, head_dim=HD,
                                     rotary_dim=rot, max_context=maxc, rope_theta=d.rope_theta,
                                     eps=d.rms_norm_eps, ld_qkv=ld)
        ws = pyq35.lib.q35_attn_prefill_workspace_bytes(args)
        if ws_min:  # no room for the pre-split tiles: the kernel splits them itself
            ws = nq * T * HD * 4 + 256
        args.qkv = B.up("rows", rows)
        args.q_norm, args.k_norm = B.up("qn", qnw), B.up("kn", knw)
        args.k_cache, args.v_cache = B.up("K", Kd), B.up("V", Vd)
        args.out = B.alloc("out", T * nq * HD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_attn_prefill(args, None))
        hip.sync()
        out = hip.download(B.p["out"], (T, nq * HD))
        Kdev = hip.download(B.p["K"], Kd.shape)
        Vdev = hip.download(B.p["V"], Vd.shape)
    finally:
        B.free()
    Ko = np.ascontiguousarray(Kd.transpose(1, 0, 2))
    Vo = np.ascontiguousarray(Vd.transpose(1, 0, 2))
    ref = np.zeros((T, nq * HD), np.float32)
    q0, k0, v0 = 0, 2 * nq * HD, 2 * nq * HD + nkv * HD
    for t in range(T):
        r = rows[t]
        ref[t] = op.attn_core(d, pos0 + t, r[q0:k0], r[k0:v0], r[v0:], qnw, knw, Ko, Vo)
    return out, ref, Kdev, Ko, Vdev, Vo


@pytest.mark.parametrize("nq,nkv,T,pos0", [
    (2, 1, 1, 0), (2, 1, 70, 0), (4, 1, 64, 0), (2, 2, 33, 0), (8, 2, 65, 37),
    (16, 2, 130, 0),      # the 2B head shape (GQA 8:1)
    (16, 2, 200, 1000),   # continuing after 1000 cached positions
])
def test_attn_prefill_vs_oracle(hip, nq, nkv, T, pos0):
    out, ref, Kdev, Ko, Vdev, Vo = run_attn_prefill(hip, nq, nkv, T, pos0, seed=T + 3 * pos0 + nq)
    errs = [rel_l2(out[t], ref[t]) for t in range(T)]
    print(f"worst per-token rel_l2 {max(errs):.3g}")
    assert max(errs) < REL_L2, f"token {int(np.argmax(errs))}: {max(errs)}"
    for kh in range(nkv):
        np.testing.assert_allclose(Kdev[kh, :pos0 + T], Ko[:pos0 + T, kh], rtol=2e-6, atol=2e-6)
        np.testing.assert_array_equal(Vdev[kh, :pos0 + T], Vo[:pos0 + T, kh])


@pytest.mark.parametrize("nq,nkv,T,pos0", [(2, 1, 70, 0), (8, 2, 65, 37), (16, 2, 300, 1000)])
def test_attn_prefill_split_tiles_match_presplit(hip, nq, nkv, T, pos0):
    """A workspace without room for the pre-split key / value tiles runs the kernel that splits
    each tile itself: the same parts and products, so the same output bit for bit, and both
    within the bar against the oracle."""
    seed = 7 * T + pos0
    out_img, ref, _, _, _, _ = run_attn_prefill(hip, nq, nkv, T, pos0, seed=seed)
    out_own, _, _, _, _, _ = run_attn_prefill(hip, nq, nkv, T, pos0, seed=seed, ws_min=True)
    np.testing.assert_array_equal(out_img, out_own)
    assert max(rel_l2(out_img[t], ref[t]) for t in range(T)) < REL_L2


@pytest.mark.parametrize("rot", [0, 18, 32, 256])
def test_attn_prefill_rotary_widths(hip, rot):
    """Rotary widths other than the model's 64: multiples of 8 take the per-token prep
    kernel, others (18) the per-dim one; 0 and the full head width are the edges."""
    out, ref, Kdev, Ko, Vdev, Vo = run_attn_prefill(hip, 8, 2, 70, 30, seed=rot + 1, rot=rot)
    errs = [rel_l2(out[t], ref[t]) for t in range(70)]
    assert max(errs) < REL_L2, f"rot {rot}: {max(errs)}"
    for kh in range(2):
        np.testing.assert_allclose(Kdev[kh, :100], Ko[:100, kh], rtol=2e-6, atol=2e-6)


# ----------------------------------------------------------------------------- model level
NAMES = ["tiny", "tiny_gqa", "tiny_untied"]


@pytest.mark.parametrize("name", NAMES)
def test_model_prefill_vs_golden(model_dirs, name):
    """Logits of every prompt row vs the reference's step logits (and, where the reference's
    QwenForward::prefill applies, its prefill logits); hidden state after every layer."""
    g = golden(name)
    m = pyq35.Model(model_dirs[name], 600)
    lg = m.prefill(g["prompt"])
    for t in range(len(g["prompt"])):
        assert rel_l2(lg[t], g["logits"][t]) < REL_L2, f"row {t}"
        if "prefill_logits" in g:
            assert rel_l2(lg[t], g["prefill_logits"][t]) < REL_L2, f"prefill row {t}"
    m.reset()
    _, tr = m.extend(g["prompt"], want_logits=False, want_trace=True)
    worst = max(rel_l2(tr[t, l], g["trace"][t, l]) for t in range(tr.shape[0]) for l in range(tr.shape[1]))
    print(f"{name}: worst per-layer rel_l2 {worst:.3g}")
    assert worst < REL_L2
    m.close()


@pytest.mark.parametrize("name", NAMES)
def test_prefill_hands_state_to_decode(model_dirs, name):
    """Prefill in blocks of 64 leaves the recurrent state, conv window and KV rows that
    token-serial steps leave, and greedy decoding continues with the reference's ids."""
    g = golden(name)
    ids = np.asarray(g["long_ids"][:200], np.int32)
    a = pyq35.Model(model_dirs[name], 600)
    b = pyq35.Model(model_dirs[name], 600)
    a.set_prefill_block(64)
    a.prefill(ids, want_logits=False)
    for t in ids:
        b.step(int(t), want_logits=False)
    assert a.position == b.position == len(ids)
    d = a.dims
    for l in range(d.n_layers_gdn):
        assert rel_l2(a.gdn_state(l), b.gdn_state(l)) < REL_L2
        assert rel_l2(a.conv_state(l), b.conv_state(l)) < REL_L2
    for l in range(d.n_layers_attn):
        Ka, Va = a.kv(l, 0, len(ids))
        Kb, Vb = b.kv(l, 0, len(ids))
        assert rel_l2(Ka, Kb) < REL_L2 and rel_l2(Va, Vb) < REL_L2
    assert rel_l2(a.hidden(), b.hidden()) < REL_L2
    # greedy continuation from the prefilled state = the golden greedy run
    a.reset()
    lg = a.prefill(g["prompt"])
    first = int(np.argmax(lg[-1]))
    rest = a.decode_greedy(first, len(g["greedy"]) - 1)
    np.testing.assert_array_equal(np.concatenate([[first], rest]), g["greedy"])
    a.close()
    b.close()


def test_prefill_block_invariance(model_dirs):
    """Blocks of 1, 17, 64 and 2048 tokens give the same logits (the block boundary carries
    state, conv window and KV rows)."""
    g = golden("tiny_untied")
    ids = np.asarray(g["long_ids"][:150], np.int32)
    m = pyq35.Model(model_dirs["tiny_untied"], 600)
    outs = []
    for blk in (2048, 64, 17, 1):
        m.set_prefill_block(blk)
        outs.append(m.prefill(ids))
    for o in outs[1:]:
        assert max(rel_l2(o[t], outs[0][t]) for t in range(len(ids))) < REL_L2
    m.close()


@pytest.mark.parametrize("exact", [False, True])
def test_prefill_2b_mixers_vs_oracle(tmp_path, exact):
    """2B mixer shapes (16 GDN heads, 16 q / 2 kv heads, H 2048) in a 4-layer model with a
    small vocabulary: 300 prompt tokens (ragged chunks, two blocks of 256) vs the oracle's
    sequential prefill, per layer and for the logits; on the default two-part fp16 GEMMs
    and with prefill_exact (three exact bf16 parts, no fp16 weight copies: a smaller prompt
    arena)."""
    d = pyq35.dims_for("2b")
    d.n_layers_total = 4
    d.vocab_size = 4096
    path = str(tmp_path / "m2b4")
    pyq35.synth_write_model(path, d, seed=3, std=0.02)
    ids = pyq35.synth_token_ids(2, d.vocab_size, 300)
    m = pyq35.Model(path, 512, prefill_block=256, prefill_exact=exact)
    arena = m.budget()["prompt_arena_bytes"]
    # the fp16 copies of the four projection matrices of the 4 layers (3 GDN + 1 attention)
    n16 = 0
    for l in range(4):
        attn = (l + 1) % 4 == 0
        n_in = (2 * 16 * 256 + 2 * 2 * 256 if attn else 2 * 2048 + 2048 + 2048 + 32) * 2048
        for n in (n_in, 2048 * (16 * 256 if attn else 2048), 2 * 6144 * 2048, 2048 * 6144):
            n16 += (n + 127) // 128 * 128 * 2
    if exact:
        ref_m = pyq35.Model(path, 512, prefill_block=256)
        assert ref_m.budget()["prompt_arena_bytes"] - arena >= n16
        ref_m.close()
    lg, tr = m.extend(ids, want_logits=True, want_trace=True)
    m.close()
    o = op.Oracle(path, 512)
    rtr = o.enable_trace(rows=len(ids))
    ref = o.prefill(ids)
    o.close()
    worst = max(rel_l2(tr[t, l], rtr[t, l]) for t in range(len(ids)) for l in range(4))
    print(f"2B-shaped ({'exact' if exact else 'two-part'}): worst per-layer rel_l2 {worst:.3g}")
    assert worst < REL_L2
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < REL_L2
