"""The CPU oracle against the golden vectors written from the compiled reference engine
(tests/golden/make_golden.py). These pin oracle/oracle.c before it is used as the checker
of the HIP path."""
import os

import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, golden, layer_name, rel_l2, sha256

# The oracle keeps the reference's arithmetic (order of the matvec accumulation, double
# sums in the norms, double RoPE angles), so it is held to a bar ten times tighter than
# the one the HIP path is held to.
ORACLE_BAR = REL_L2 / 10

NAMES = ["tiny", "tiny_gqa", "tiny_untied"]


@pytest.mark.parametrize("name", NAMES)
def test_checkpoint_bytes(model_dirs, name):
    """The synthetic writer reproduces the checkpoint the fixtures were made from."""
    assert sha256(model_dirs[name] + "/model.safetensors") == str(golden(name)["sha256"])


@pytest.mark.parametrize("name", NAMES)
def test_prompt_logits_and_layers(model_dirs, name):
    g = golden(name)
    o = op.Oracle(model_dirs[name], 600)
    trace = o.enable_trace()
    for t, tok in enumerate(g["prompt"]):
        lg = o.step(int(tok))
        assert rel_l2(lg, g["logits"][t]) < ORACLE_BAR, f"logits step {t}"
        for l in range(o.dims.n_layers_total):
            assert rel_l2(trace[0, l], g["trace"][t, l]) < ORACLE_BAR, f"step {t} layer {l}"
    o.close()


@pytest.mark.parametrize("name", NAMES)
def test_greedy(model_dirs, name):
    g = golden(name)
    o = op.Oracle(model_dirs[name], 600)
    ids = o.generate_greedy(g["prompt"], len(g["greedy"]))
    np.testing.assert_array_equal(ids, g["greedy"])


@pytest.mark.parametrize("name", NAMES)
def test_state_after_512_steps(model_dirs, name):
    g = golden(name)
    o = op.Oracle(model_dirs[name], 600)
    for t in g["long_ids"]:
        lg = o.step(int(t))
    assert rel_l2(o.gdn_state(0), g["S512"]) < ORACLE_BAR
    assert rel_l2(o.conv_state(0), g["W512"]) < ORACLE_BAR
    K = o.kcache(0)[:512]
    V = o.vcache(0)[:512]
    assert rel_l2(K[-8:], g["K512_last"]) < ORACLE_BAR
    assert rel_l2(V[-8:], g["V512_last"]) < ORACLE_BAR
    assert rel_l2(K.sum(axis=(1, 2)), g["K512_sum"]) < ORACLE_BAR
    assert rel_l2(lg, g["logits512"]) < ORACLE_BAR
    assert rel_l2(o.hidden(), g["hidden512"]) < ORACLE_BAR


def _mixer_weights(o, d, layer):
    H = d.hidden_size
    conv = 2 * d.gdn_k_heads * 128 + d.gdn_v_heads * 128
    vd = d.gdn_v_heads * 128
    w = {}
    if (layer + 1) % d.attn_interval:
        p = "linear_attn."
        w["in_qkv"] = o.weight_bf16(layer_name(layer, p + "in_proj_qkv.weight"), (conv, H))
        w["in_z"] = o.weight_bf16(layer_name(layer, p + "in_proj_z.weight"), (vd, H))
        w["in_b"] = o.weight_bf16(layer_name(layer, p + "in_proj_b.weight"), (d.gdn_v_heads, H))
        w["in_a"] = o.weight_bf16(layer_name(layer, p + "in_proj_a.weight"), (d.gdn_v_heads, H))
        w["out"] = o.weight_bf16(layer_name(layer, p + "out_proj.weight"), (H, vd))
        w["conv1d"] = o.weight_f32(layer_name(layer, p + "conv1d.weight"), (conv * 4,))
        w["dt_bias"] = o.weight_f32(layer_name(layer, p + "dt_bias"), (d.gdn_v_heads,))
        w["A_log"] = o.weight_f32(layer_name(layer, p + "A_log"), (d.gdn_v_heads,))
        w["norm"] = o.weight_f32(layer_name(layer, p + "norm.weight"), (128,))
    else:
        p = "self_attn."
        NQ, NKV = d.attn_q_heads, d.attn_kv_heads
        w["q"] = o.weight_bf16(layer_name(layer, p + "q_proj.weight"), (2 * NQ * 256, H))
        w["k"] = o.weight_bf16(layer_name(layer, p + "k_proj.weight"), (NKV * 256, H))
        w["v"] = o.weight_bf16(layer_name(layer, p + "v_proj.weight"), (NKV * 256, H))
        w["o"] = o.weight_bf16(layer_name(layer, p + "o_proj.weight"), (H, NQ * 256))
        w["q_norm"] = o.weight_f32(layer_name(layer, p + "q_norm.weight"), (256,))
        w["k_norm"] = o.weight_f32(layer_name(layer, p + "k_norm.weight"), (256,))
    return w


def oracle_gdn_mixer(o, d, w, x, S, win):
    qkv = op.matmul_bf16(w["in_qkv"], x)
    z = op.matmul_bf16(w["in_z"], x)
    b = op.matmul_bf16(w["in_b"], x)
    a = op.matmul_bf16(w["in_a"], x)
    _, gn = op.gdn_core(d, qkv, z, b, a, w["conv1d"], w["A_log"], w["dt_bias"], w["norm"], win, S)
    return op.matmul_bf16(w["out"], gn)


def oracle_attn_mixer(o, d, w, x, pos, K, V):
    qg = op.matmul_bf16(w["q"], x)
    kn = op.matmul_bf16(w["k"], x)
    vn = op.matmul_bf16(w["v"], x)
    ac = op.attn_core(d, pos, qg, kn, vn, w["q_norm"], w["k_norm"], K, V)
    return op.matmul_bf16(w["o"], ac)


@pytest.mark.parametrize("name", NAMES)
def test_single_mixers(model_dirs, name):
    """One reference gdn_step / attn_step on injected state, restated by the oracle's
    matvec + gdn_core / attn_core."""
    g = golden(name)
    o = op.Oracle(model_dirs[name], 600)
    d = o.dims
    w = _mixer_weights(o, d, 0)
    S = g["gdn_S0"].copy()
    win = g["gdn_W0"].copy()
    out = oracle_gdn_mixer(o, d, w, g["gdn_in"], S, win)
    assert rel_l2(out, g["gdn_out"]) < ORACLE_BAR
    assert rel_l2(S, g["gdn_S1"]) < ORACLE_BAR
    np.testing.assert_array_equal(win, g["gdn_W1"])

    al = d.attn_interval - 1
    w = _mixer_weights(o, d, al)
    pos = g["attn_K0"].shape[0]
    K = np.zeros((pos + 1, d.attn_kv_heads, 256), np.float32)
    V = np.zeros_like(K)
    K[:pos] = g["attn_K0"]
    V[:pos] = g["attn_V0"]
    out = oracle_attn_mixer(o, d, w, g["attn_in"], pos, K, V)
    assert rel_l2(out, g["attn_out"]) < ORACLE_BAR
    assert rel_l2(K[pos], g["attn_krow"]) < ORACLE_BAR
    np.testing.assert_array_equal(V[pos], g["attn_vrow"])


def test_prefill_logits(model_dirs):
    g = golden("tiny")
    o = op.Oracle(model_dirs["tiny"], 600)
    lg = o.prefill(g["prompt"])
    assert rel_l2(lg, g["prefill_logits"]) < ORACLE_BAR
    # the reference's stateless prefill and its token-serial decode agree
    assert rel_l2(g["prefill_logits"], g["logits"]) < REL_L2


@pytest.mark.parametrize("name", ["tiny", "tiny_untied"])
def test_prefill_handoff_equals_token_serial_steps(model_dirs, name):
    """The oracle's prefill with handoff on leaves exactly the state that token-serial steps
    leave (GDN state, conv window, K / V rows, residual, position): the prefill and the step
    restate the same reference arithmetic (src/qwen_forward.cpp:83-152 and
    src/qwen_model.cpp:154-209 share their loops), so the two agree bit for bit."""
    ids = pyq35.synth_token_ids(1, pyq35.dims_for(name).vocab_size, 150)
    a = op.Oracle(model_dirs[name], 200)
    a.set_prefill_handoff(True)
    a.prefill(ids, want_logits=False)
    b = op.Oracle(model_dirs[name], 200)
    for t in ids:
        b.step(int(t))
    assert a.position == b.position == len(ids)
    d = a.dims
    n_gdn = d.n_layers_total - d.n_layers_total // d.attn_interval
    for i in range(n_gdn):
        np.testing.assert_array_equal(a.gdn_state(i), b.gdn_state(i))
        np.testing.assert_array_equal(a.conv_state(i), b.conv_state(i))
    for l in range(d.n_layers_total // d.attn_interval):
        np.testing.assert_array_equal(a.kcache(l)[:len(ids)], b.kcache(l)[:len(ids)])
        np.testing.assert_array_equal(a.vcache(l)[:len(ids)], b.vcache(l)[:len(ids)])
    np.testing.assert_array_equal(a.hidden(), b.hidden())
    np.testing.assert_array_equal(a.step(int(ids[0])), b.step(int(ids[0])))
    a.close()
    b.close()


def test_untied_prefill_uses_the_embedding_head(model_dirs):
    """QwenForward::prefill's output head is the embedding over all its rows even when the
    checkpoint has an lm_head (src/qwen_forward.cpp:193-199): the oracle's prefill equals the
    reference's on the untied checkpoint, and differs from the step's logits (lm_head)."""
    g = golden("untied_prefill")
    assert sha256(os.path.join(model_dirs["tiny_untied"], "model.safetensors")) == str(g["sha256"])
    o = op.Oracle(model_dirs["tiny_untied"], 64)
    lg = o.prefill(g["prompt"])
    o.reset()
    step = np.stack([o.step(int(t)) for t in g["prompt"]])
    o.close()
    assert rel_l2(lg, g["prefill_logits"]) < 1e-6
    assert rel_l2(step, g["step_logits"]) < 1e-6
    assert rel_l2(g["prefill_logits"], g["step_logits"]) > 0.5
