"""The two decode mixer kernels through the kernel-level C ABI (q35_gdn_decode,
q35_attn_decode) against the oracle's gdn_core / attn_core on the same seeded inputs:
the isolated-GDN and attention-decode workloads (16 heads of 128 x 128 fp32 state; GQA 8:1
over an fp32 cache at 2k/8k/32k) plus edge cases."""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, rel_l2, ring_from_window, window_from_ring

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    return pyq35.Hip()


class Bufs:
    def __init__(self, hip):
        self.hip, self.p = hip, {}

    def up(self, name, a):
        if name in self.p:
            self.hip.copy_in(self.p[name], a)
        else:
            self.p[name] = self.hip.upload(a)
        return self.p[name]

    def alloc(self, name, nbytes):
        self.p[name] = self.hip.malloc(nbytes)
        return self.p[name]

    def free(self):
        for v in self.p.values():
            self.hip.free(v)
        self.p = {}


def gdn_dims(kh, vh):
    return pyq35.default_dims(gdn_k_heads=kh, gdn_v_heads=vh)


@pytest.mark.parametrize("kh,vh,layers,steps,fused", [
    (16, 16, 2, 512, False),   # the isolated-GDN shape, 512 steps (state bar after 512 steps)
    (16, 16, 3, 24, True),     # gated norm fused in the kernel (one workgroup per head)
    (8, 16, 2, 40, False),     # v-heads = 2 k-heads: q/k shared by two v-heads
    (16, 16, 18, 24, False),   # 18 layers per launch: 64-column slices (576 workgroups)
    (8, 16, 16, 16, False),    # 64-column slices with q/k shared by two v-heads
])
def test_gdn_decode_vs_oracle(hip, kh, vh, layers, steps, fused):
    rng = np.random.default_rng(100 + kh + vh + steps)
    d = gdn_dims(kh, vh)
    KD, VD = kh * 128, vh * 128
    CONV = 2 * KD + VD
    conv_w = (0.5 * rng.standard_normal((layers, CONV * 4))).astype(np.float32)
    A_log = rng.standard_normal((layers, vh)).astype(np.float32)
    dt_bias = rng.standard_normal((layers, vh)).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal((layers, 128))).astype(np.float32)
    S = (0.1 * rng.standard_normal((layers, vh, 128, 128))).astype(np.float32)
    win = rng.standard_normal((layers, CONV, 3)).astype(np.float32)
    pos0 = 5
    B = Bufs(hip)
    try:
        B.up("conv_w", conv_w)
        B.up("A_log", A_log)
        B.up("dt_bias", dt_bias)
        B.up("norm_w", norm_w)
        B.up("state", S)
        B.up("ring", np.stack([ring_from_window(win[l], pos0) for l in range(layers)]))
        B.alloc("out", layers * VD * 4)
        S_o = S.copy()
        win_o = win.copy()
        worst = 0.0
        for t in range(steps):
            pos = pos0 + t
            qkv = rng.standard_normal((layers, CONV)).astype(np.float32)
            z = rng.standard_normal((layers, VD)).astype(np.float32)
            b = rng.standard_normal((layers, vh)).astype(np.float32)
            a = rng.standard_normal((layers, vh)).astype(np.float32)
            args = pyq35.GdnDecodeArgs(
                n_layers=layers, k_heads=kh, v_heads=vh, head_dim_k=128, head_dim_v=128,
                conv_kernel=4, pos=pos, eps=d.rms_norm_eps, qkv=B.up("qkv", qkv), z=B.up("z", z),
                b=B.up("b", b), a=B.up("a", a), conv_w=B.p["conv_w"], A_log=B.p["A_log"],
                dt_bias=B.p["dt_bias"], norm_w=B.p["norm_w"] if fused else None,
                conv_ring=B.p["ring"], state=B.p["state"], out=B.p["out"])
            pyq35.check(pyq35.lib.q35_gdn_decode(args, None))
            hip.sync()
            out = hip.download(B.p["out"], (layers, VD))
            for l in range(layers):
                raw, normed = op.gdn_core(d, qkv[l], z[l], b[l], a[l], conv_w[l], A_log[l],
                                          dt_bias[l], norm_w[l], win_o[l], S_o[l])
                ref = normed if fused else raw
                e = rel_l2(out[l], ref)
                worst = max(worst, e)
                assert e < REL_L2, f"step {t} layer {l}: {e}"
        S_dev = hip.download(B.p["state"], S.shape)
        ring = hip.download(B.p["ring"], (layers, 4, CONV))
    finally:
        B.free()
    for l in range(layers):
        assert rel_l2(S_dev[l], S_o[l]) < REL_L2
        np.testing.assert_array_equal(window_from_ring(ring[l], pos0 + steps), win_o[l])
    print(f"worst per-step output rel_l2 {worst:.3g}, state rel_l2 "
          f"{max(rel_l2(S_dev[l], S_o[l]) for l in range(layers)):.3g}")


def attn_dims(nq, nkv):
    return pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)


def run_attn(hip, nq, nkv, pos, max_ctx, n_splits, seed, rot=64):
    rng = np.random.default_rng(seed)
    d = attn_dims(nq, nkv)
    d.partial_rotary_factor = rot / 256.0
    HD = 256
    qg = rng.standard_normal(2 * nq * HD).astype(np.float32)
    kn = rng.standard_normal(nkv * HD).astype(np.float32)
    vn = rng.standard_normal(nkv * HD).astype(np.float32)
    qnw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    knw = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    Kd = np.zeros((nkv, max_ctx, HD), np.float32)  # device layout [NKV][ctx][HD]
    Vd = np.zeros_like(Kd)
    Kd[:, :pos] = rng.standard_normal((nkv, pos, HD))
    Vd[:, :pos] = rng.standard_normal((nkv, pos, HD))
    B = Bufs(hip)
    try:
        args = pyq35.AttnDecodeArgs(q_heads=nq, kv_heads=nkv, head_dim=HD, rotary_dim=rot, pos=pos,
                                    n_splits=n_splits, max_context=max_ctx, rope_theta=d.rope_theta,
                                    eps=d.rms_norm_eps)
        ws = pyq35.lib.q35_attn_decode_workspace_bytes(args)
        args.qg, args.k_new, args.v_new = B.up("qg", qg), B.up("kn", kn), B.up("vn", vn)
        args.q_norm, args.k_norm = B.up("qnw", qnw), B.up("knw", knw)
        args.k_cache, args.v_cache = B.up("K", Kd), B.up("V", Vd)
        args.out = B.alloc("out", nq * HD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_attn_decode(args, None))
        hip.sync()
        out = hip.download(B.p["out"], nq * HD)
        Kdev = hip.download(B.p["K"], Kd.shape)
        Vdev = hip.download(B.p["V"], Vd.shape)
    finally:
        B.free()
    Ko = np.ascontiguousarray(Kd.transpose(1, 0, 2))
    Vo = np.ascontiguousarray(Vd.transpose(1, 0, 2))
    ref = op.attn_core(d, pos, qg, kn, vn, qnw, knw, Ko, Vo)
    return out, ref, Kdev[:, pos], Ko[pos], Vdev[:, pos], Vo[pos]


@pytest.mark.parametrize("nq,nkv", [(16, 2), (8, 2), (2, 1), (4, 1), (2, 2), (16, 1)])
@pytest.mark.parametrize("pos", [0, 1, 31, 32, 33, 64, 100])
def test_attn_decode_small(hip, nq, nkv, pos):
    out, ref, krow, kref, vrow, vref = run_attn(hip, nq, nkv, pos, pos + 3, 0, seed=pos * 31 + nq)
    assert rel_l2(out, ref) < REL_L2
    np.testing.assert_allclose(krow, kref, rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(vrow, vref)


@pytest.mark.parametrize("pos", [2047, 8191, 32767, 131071])
def test_attn_decode_2b_shape(hip, pos):
    """16 q heads / 2 kv heads (GQA 8:1), head_dim 256, partial RoPE 64, at 2k/8k/32k and the
    longest context of the long-decode workload (131072 positions, 1 GiB of K/V)."""
    out, ref, krow, kref, vrow, vref = run_attn(hip, 16, 2, pos, pos + 1, 0, seed=pos)
    assert rel_l2(out, ref) < REL_L2
    np.testing.assert_allclose(krow, kref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("rot", [0, 18, 32, 96, 256])
def test_attn_decode_rotary_widths(hip, rot):
    """GQA 8 with rotary widths that are multiples of 32 takes the matrix-core kernel, others
    (18) the vector-ALU kernel; 0 and the full head width are the edges."""
    out, ref, krow, kref, *_ = run_attn(hip, 16, 2, 500, 600, 0, seed=rot + 7, rot=rot)
    assert rel_l2(out, ref) < REL_L2
    np.testing.assert_allclose(krow, kref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("n_splits", [1, 3, 64, 1024])
def test_attn_decode_split_invariance(hip, n_splits):
    """The split-K combine equals the single-pass softmax for any number of splits."""
    out, ref, *_ = run_attn(hip, 16, 2, 3000, 4096, n_splits, seed=77)
    assert rel_l2(out, ref) < REL_L2


# (pos, n_splits) -> positions per split of the matrix-core kernel (four waves of 16-position
# tiles): 8192 / 8263 over 128: 65 per split (a second, one-position tile), the last split 3
# positions; 9200: 72 per split; 9700: 76; 130 over 2: 66 and 65; 9 over 4: 3 per split
@pytest.mark.parametrize("pos,n_splits", [(8192, 128), (8263, 128), (9200, 128), (9700, 128), (130, 2), (9, 4)])
def test_attn_decode_split_shapes(hip, pos, n_splits):
    """Splits just past a multiple of the tile, ragged last splits and splits shorter than a
    tile, against the oracle."""
    out, ref, krow, kref, vrow, vref = run_attn(hip, 16, 2, pos, pos + 1, n_splits, seed=pos + n_splits)
    assert rel_l2(out, ref) < REL_L2
    np.testing.assert_allclose(krow, kref, rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(vrow, vref)


@pytest.mark.parametrize("L,nq,nkv,pos,maxc", [
    (3, 8, 2, 700, 800),      # vector-ALU kernel (GQA 4)
    (6, 16, 2, 8200, 8300),   # matrix-core kernel, 6 layers at 8k: two workgroups per CU (42 splits)
])
def test_attn_decode_layer_batch(hip, L, nq, nkv, pos, maxc):
    """Independent layers in one launch (grid.z) equal one oracle call per layer."""
    rng = np.random.default_rng(5)
    HD = 256
    d = attn_dims(nq, nkv)
    qg = rng.standard_normal((L, 2 * nq * HD)).astype(np.float32)
    kn = rng.standard_normal((L, nkv * HD)).astype(np.float32)
    vn = rng.standard_normal((L, nkv * HD)).astype(np.float32)
    qw = (0.1 * rng.standard_normal((L, HD))).astype(np.float32)
    kw = (0.1 * rng.standard_normal((L, HD))).astype(np.float32)
    Kd = np.zeros((L, nkv, maxc, HD), np.float32)
    Vd = np.zeros_like(Kd)
    Kd[:, :, :pos] = rng.standard_normal((L, nkv, pos, HD))
    Vd[:, :, :pos] = rng.standard_normal((L, nkv, pos, HD))
    B = Bufs(hip)
    try:
        args = pyq35.AttnDecodeArgs(q_heads=nq, kv_heads=nkv, head_dim=HD, rotary_dim=64, pos=pos,
                                    n_splits=0, n_layers=L, max_context=maxc, rope_theta=d.rope_theta,
                                    eps=d.rms_norm_eps)
        ws = pyq35.lib.q35_attn_decode_workspace_bytes(args)
        args.qg, args.k_new, args.v_new = B.up("qg", qg), B.up("kn", kn), B.up("vn", vn)
        args.q_norm, args.k_norm = B.up("qw", qw), B.up("kw", kw)
        args.k_cache, args.v_cache = B.up("K", Kd), B.up("V", Vd)
        args.out = B.alloc("out", L * nq * HD * 4)
        args.workspace = B.alloc("ws", ws)
        args.workspace_bytes = ws
        pyq35.check(pyq35.lib.q35_attn_decode(args, None))
        hip.sync()
        out = hip.download(B.p["out"], (L, nq * HD))
        Kdev = hip.download(B.p["K"], Kd.shape)
    finally:
        B.free()
    for l in range(L):
        Ko = np.ascontiguousarray(Kd[l].transpose(1, 0, 2))
        Vo = np.ascontiguousarray(Vd[l].transpose(1, 0, 2))
        ref = op.attn_core(d, pos, qg[l], kn[l], vn[l], qw[l], kw[l], Ko, Vo)
        assert rel_l2(out[l], ref) < REL_L2, f"layer {l}"
        np.testing.assert_allclose(Kdev[l, :, pos], Ko[pos], rtol=2e-6, atol=2e-6)
