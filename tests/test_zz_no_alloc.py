"""q35_attn_decode_static, the attention decode that allocates nothing (its split-K partials
live in the library's static device array), against q35_attn_decode with a caller workspace:
two calls in a row -- the second smaller, so partials a larger call left behind must not
leak into it -- each compared bit for bit with the workspace entry point on the same inputs,
and against the oracle; the library makes no device allocation for these calls. (The refusal
of partials beyond the static array is host logic, tested in test_c_abi.py.)"""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, rel_l2

pytestmark = pytest.mark.gpu

HD = 256


@pytest.fixture(scope="module")
def hip():
    return pyq35.Hip()


def make_inputs(nq, nkv, n_layers, pos, max_ctx, seed):
    rng = np.random.default_rng(seed)
    L = n_layers
    x = {
        "qg": rng.standard_normal((L, 2 * nq * HD)).astype(np.float32),
        "kn": rng.standard_normal((L, nkv * HD)).astype(np.float32),
        "vn": rng.standard_normal((L, nkv * HD)).astype(np.float32),
        "qw": (0.1 * rng.standard_normal((L, HD))).astype(np.float32),
        "kw": (0.1 * rng.standard_normal((L, HD))).astype(np.float32),
        "K": np.zeros((L, nkv, max_ctx, HD), np.float32),
        "V": np.zeros((L, nkv, max_ctx, HD), np.float32),
    }
    x["K"][:, :, :pos] = rng.standard_normal((L, nkv, pos, HD))
    x["V"][:, :, :pos] = rng.standard_normal((L, nkv, pos, HD))
    return x


def run(hip, entry, x, nq, nkv, n_layers, pos, max_ctx, rot=64):
    """One call of `entry` on fresh device copies of the inputs: (out, K, V) afterwards."""
    d = pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)
    bufs = {k: hip.upload(np.ascontiguousarray(v)) for k, v in x.items()}
    out = hip.malloc(n_layers * nq * HD * 4)
    ws = None
    try:
        args = pyq35.AttnDecodeArgs(q_heads=nq, kv_heads=nkv, head_dim=HD, rotary_dim=rot, pos=pos,
                                    n_splits=0, n_layers=n_layers, max_context=max_ctx,
                                    rope_theta=d.rope_theta, eps=d.rms_norm_eps)
        args.qg, args.k_new, args.v_new = bufs["qg"], bufs["kn"], bufs["vn"]
        args.q_norm, args.k_norm = bufs["qw"], bufs["kw"]
        args.k_cache, args.v_cache, args.out = bufs["K"], bufs["V"], out
        if entry == "workspace":
            n = pyq35.lib.q35_attn_decode_workspace_bytes(args)
            ws = hip.malloc(n)
            args.workspace, args.workspace_bytes = ws, n
            pyq35.check(pyq35.lib.q35_attn_decode(args, None))
        else:
            pyq35.check(pyq35.lib.q35_attn_decode_static(args, None))
        hip.sync()
        return (hip.download(out, (n_layers, nq * HD)), hip.download(bufs["K"], x["K"].shape),
                hip.download(bufs["V"], x["V"].shape))
    finally:
        for p in list(bufs.values()) + [out] + ([ws] if ws else []):
            hip.free(p)


def oracle_out(x, nq, nkv, l, pos):
    d = pyq35.default_dims(attn_q_heads=nq, attn_kv_heads=nkv)
    Ko = np.ascontiguousarray(x["K"][l].transpose(1, 0, 2))
    Vo = np.ascontiguousarray(x["V"][l].transpose(1, 0, 2))
    return op.attn_core(d, pos, x["qg"][l], x["kn"][l], x["vn"][l], x["qw"][l], x["kw"][l], Ko, Vo)


# (q heads, kv heads, layers per call, position, max context): the 2B head shape on the
# matrix-core kernel, a large call then a smaller one, then the vector-ALU kernel (GQA 4)
CALLS = [(16, 2, 2, 8000, 8192), (16, 2, 1, 300, 1024), (8, 2, 1, 2000, 4096)]


def test_static_scratch_matches_workspace_entry(hip):
    allocs = pyq35.lib.q35_device_alloc_count()
    for i, (nq, nkv, L, pos, max_ctx) in enumerate(CALLS):
        print(f"call {i}: q_heads {nq} kv_heads {nkv} layers {L} position {pos} max_context {max_ctx}", flush=True)
        x = make_inputs(nq, nkv, L, pos, max_ctx, seed=100 + i)
        o_ws, K_ws, V_ws = run(hip, "workspace", x, nq, nkv, L, pos, max_ctx)
        o_st, K_st, V_st = run(hip, "static", x, nq, nkv, L, pos, max_ctx)
        np.testing.assert_array_equal(o_st, o_ws)
        np.testing.assert_array_equal(K_st, K_ws)
        np.testing.assert_array_equal(V_st, V_ws)
        for l in range(L):
            assert rel_l2(o_st[l], oracle_out(x, nq, nkv, l, pos)) < REL_L2
    assert pyq35.lib.q35_device_alloc_count() == allocs

