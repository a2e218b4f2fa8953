"""The device decoder (q35_model_*) against the golden vectors of the compiled reference and
against the oracle: logits and residual stream after every layer, greedy ids, recurrent state
and KV rows after 512 steps, the 0.8B-shaped full greedy decode, graph replay, the
zero-allocation step and the error paths."""
import json
import os
import tempfile

import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, golden, rel_l2, sha256

pytestmark = pytest.mark.gpu
NAMES = ["tiny", "tiny_gqa", "tiny_untied"]


@pytest.mark.parametrize("name", NAMES)
def test_prompt_logits_and_layers(model_dirs, name):
    g = golden(name)
    m = pyq35.Model(model_dirs[name], 600)
    m.set_layer_trace(True)
    worst = 0.0
    for t, tok in enumerate(g["prompt"]):
        lg, _ = m.step(int(tok))
        assert rel_l2(lg, g["logits"][t]) < REL_L2, f"logits step {t}"
        tr = m.layer_trace()
        for l in range(tr.shape[0]):
            e = rel_l2(tr[l], g["trace"][t, l])
            worst = max(worst, e)
            assert e < REL_L2, f"step {t} layer {l}: {e}"
    print(f"{name}: worst per-layer rel_l2 {worst:.3g}")
    m.close()


@pytest.mark.parametrize("name", NAMES)
def test_greedy_ids(model_dirs, name):
    g = golden(name)
    m = pyq35.Model(model_dirs[name], 600)
    ids = m.generate_greedy(g["prompt"], len(g["greedy"]))
    np.testing.assert_array_equal(ids, g["greedy"])
    m.close()


@pytest.mark.parametrize("name", NAMES)
def test_state_after_512_steps(model_dirs, name):
    g = golden(name)
    m = pyq35.Model(model_dirs[name], 600)
    for t in g["long_ids"]:
        lg, _ = m.step(int(t))
    assert rel_l2(m.gdn_state(0), g["S512"]) < REL_L2
    # the window holds in_proj_qkv outputs of the last three tokens (fp32 matvec results)
    assert rel_l2(m.conv_state(0), g["W512"]) < REL_L2
    K, V = m.kv(0, 0, 512)
    assert rel_l2(K[-8:], g["K512_last"]) < REL_L2
    assert rel_l2(V[-8:], g["V512_last"]) < REL_L2
    assert rel_l2(K.sum(axis=(1, 2)), g["K512_sum"]) < REL_L2
    assert rel_l2(V.sum(axis=(1, 2)), g["V512_sum"]) < REL_L2
    assert rel_l2(lg, g["logits512"]) < REL_L2
    assert rel_l2(m.hidden(), g["hidden512"]) < REL_L2
    m.close()


def test_graph_replay_matches_eager(model_dirs):
    g = golden("tiny_untied")
    m = pyq35.Model(model_dirs["tiny_untied"], 600)
    res = []
    for graph in (False, True, True):
        m.set_graph(graph)
        m.reset()
        res.append(np.stack([m.step(int(t))[0] for t in g["prompt"]]))
    np.testing.assert_array_equal(res[0], res[1])
    np.testing.assert_array_equal(res[1], res[2])
    # the device-side greedy loop (graph replays, no host round trip) = step-by-step argmax
    m.reset()
    for t in g["prompt"][:-1]:
        m.step(int(t))
    ids = m.decode_greedy(int(g["prompt"][-1]), 16)
    np.testing.assert_array_equal(ids, g["greedy"])
    # runs of eight steps in one graph plus single-step replays for the remainder (19 =
    # 2 x 8 + 3), then a step after them: the same ids and logits as the eager loop
    out = []
    for graph in (False, True):
        m.set_graph(graph)
        m.reset()
        ids = m.decode_greedy(int(g["prompt"][0]), 19)
        out.append((ids, m.step(int(ids[-1]))[0], m.position))
    np.testing.assert_array_equal(out[0][0], out[1][0])
    np.testing.assert_array_equal(out[0][1], out[1][1])
    assert out[0][2] == out[1][2] == 20
    m.close()


def test_step_allocates_nothing(model_dirs):
    m = pyq35.Model(model_dirs["tiny"], 600)
    before = pyq35.lib.q35_device_alloc_count()
    for graph in (False, True):
        m.set_graph(graph)
        for t in range(20):
            m.step(t)
        m.decode_greedy(3, 10)
    m.reset()
    assert pyq35.lib.q35_device_alloc_count() == before
    b = m.budget()
    assert b["kv_cache_bytes"] == 1 * 2 * 1 * 600 * 256 * 4
    assert b["gdn_state_bytes"] == 3 * 2 * 128 * 128 * 4
    m.close()


def test_error_paths(model_dirs):
    m = pyq35.Model(model_dirs["tiny"], 4)
    with pytest.raises(pyq35.Q35Error) as e:
        m.step(1024)
    assert e.value.status == -6
    with pytest.raises(pyq35.Q35Error):
        m.step(-1)
    for t in range(4):
        m.step(t)
    with pytest.raises(pyq35.Q35Error) as e:
        m.step(0)
    assert e.value.status == -6 and m.position == 4
    with pytest.raises(pyq35.Q35Error):
        m.decode_greedy(0, 1)
    m.reset()
    assert m.position == 0
    m.step(0)
    m.close()


def test_state_import_then_step_matches_oracle(model_dirs):
    """Write a random state in the reference layouts, step once on both sides."""
    rng = np.random.default_rng(3)
    d = pyq35.dims_for("tiny")
    m = pyq35.Model(model_dirs["tiny"], 64)
    o = op.Oracle(model_dirs["tiny"], 64)
    pos = 9
    m.set_position(pos)
    o.set_position(pos)
    conv = 2 * d.gdn_k_heads * 128 + d.gdn_v_heads * 128
    for l in range(d.n_layers_gdn):
        S = (0.1 * rng.standard_normal((d.gdn_v_heads, 128, 128))).astype(np.float32)
        W = rng.standard_normal((conv, 3)).astype(np.float32)
        m.set_gdn_state(l, S)
        m.set_conv_state(l, W)
        np.testing.assert_array_equal(m.gdn_state(l), S)
        np.testing.assert_array_equal(m.conv_state(l), W)
        o.gdn_state(l)[:] = S
        o.conv_state(l)[:] = W
    K = rng.standard_normal((pos, d.attn_kv_heads, 256)).astype(np.float32)
    V = rng.standard_normal((pos, d.attn_kv_heads, 256)).astype(np.float32)
    m.set_kv(0, 0, K, V)
    Kb, Vb = m.kv(0, 0, pos)
    np.testing.assert_array_equal(Kb, K)
    np.testing.assert_array_equal(Vb, V)
    o.kcache(0)[:pos] = K
    o.vcache(0)[:pos] = V
    lg, _ = m.step(5)
    ref = o.step(5)
    assert rel_l2(lg, ref) < REL_L2
    assert rel_l2(m.gdn_state(0), o.gdn_state(0)) < REL_L2
    # the window shifted by one: the two older inputs were imported, the newest is the
    # in_proj_qkv output of this step
    win = m.conv_state(0)
    np.testing.assert_array_equal(win[:, :2], o.conv_state(0)[:, :2])
    assert rel_l2(win[:, 2], o.conv_state(0)[:, 2]) < REL_L2
    m.close()


def test_fill_synthetic(model_dirs):
    m = pyq35.Model(model_dirs["tiny"], 4096)
    m.fill_synthetic(4000, seed=11, state_std=0.1)
    assert m.position == 4000
    K, V = m.kv(0, 0, 4000)
    assert abs(K.mean()) < 0.01 and abs(K.std() - 1) < 0.01 and abs(V.std() - 1) < 0.01
    assert not np.array_equal(K, V)
    S = m.gdn_state(1)
    assert abs(S.std() - 0.1) < 0.002
    assert (m.conv_state(2) == 0).all()
    m.step(1)
    assert m.position == 4001
    m.close()


def test_prefill_logits_match_reference(model_dirs):
    g = golden("tiny")
    m = pyq35.Model(model_dirs["tiny"], 600)
    lg = m.prefill(g["prompt"])
    assert rel_l2(lg, g["prefill_logits"]) < REL_L2
    assert m.position == len(g["prompt"])
    m.close()


@pytest.fixture(scope="module")
def c1_dir():
    d = pyq35.dims_for("0.8b")
    root = tempfile.mkdtemp(prefix="q35_c1_")
    path = os.path.join(root, "m")
    pyq35.synth_write_model(path, d, seed=0, std=0.02, threads=16)
    yield path
    for f in os.listdir(path):
        os.remove(os.path.join(path, f))
    os.rmdir(path)
    os.rmdir(root)


def test_c1_08b_greedy_decode(c1_dir):
    """0.8B-shaped model, 32-token prompt (seed 1), 128 greedy steps: token-exact against
    the reference; residual stream after every layer and the top logits at three positions."""
    g = golden("c1_08b")
    assert sha256(os.path.join(c1_dir, "model.safetensors")) == str(g["sha256"])
    prompt, greedy = g["prompt"], g["greedy"]
    m = pyq35.Model(c1_dir, len(prompt) + len(greedy) + 2)
    ids = m.generate_greedy(prompt, len(greedy))
    np.testing.assert_array_equal(ids, greedy)
    seq = np.concatenate([prompt, greedy[:-1]])
    record = list(g["record"])
    m.reset()
    m.set_layer_trace(True)
    worst = 0.0
    for t, tok in enumerate(seq):
        lg, _ = m.step(int(tok), want_logits=t in record)
        if t in record:
            i = record.index(t)
            tr = m.layer_trace()
            for l in range(tr.shape[0]):
                e = rel_l2(tr[l], g["trace"][i, l])
                worst = max(worst, e)
                assert e < REL_L2, f"position {t} layer {l}: {e}"
            np.testing.assert_array_equal(np.argsort(-lg, kind="stable")[:4], g["top_idx"][i][:4])
            np.testing.assert_allclose(lg[g["top_idx"][i]], g["top_val"][i], rtol=1e-4, atol=1e-4)
    print(f"0.8b worst per-layer rel_l2 {worst:.3g}")
    m.close()


def test_cpp_cli_generate(model_dirs):
    """The C++ drop-in (SafeTensors + QwenModel, reference CLI flow) through lib/q35_generate."""
    import subprocess

    import pyq35 as _p

    g = golden("tiny_untied")
    exe = os.path.join(os.path.dirname(_p.LIB_PATH), "q35_generate")
    ids = ",".join(str(int(t)) for t in g["prompt"])
    out = subprocess.run([exe, model_dirs["tiny_untied"], str(len(g["greedy"])), ids], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    got = [int(x) for x in out.stdout.strip().split(",")]
    assert got == g["greedy"].tolist()


def test_prefill_wide_ffn_matches_decode(tmp_path):
    """A gate/up projection 12288 wide takes the 128 x 256 GEMM tiles (with the SwiGLU
    epilogue) and a 200-token prompt is a ragged row count: the prefill logits equal the
    token-by-token decode logits (the matvec path, itself checked against the oracle)."""
    d = pyq35.default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                           attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=6144,
                           vocab_size=1024, native_max_context=4096)
    path = str(tmp_path / "wide")
    pyq35.synth_write_model(path, d, seed=3, std=0.02)
    prompt = pyq35.synth_token_ids(5, d.vocab_size, 200)
    m = pyq35.Model(path, 256)
    lg = m.prefill(prompt)
    m.close()
    m = pyq35.Model(path, 256)
    ref = np.stack([m.step(int(t))[0] for t in prompt])
    m.close()
    assert rel_l2(lg, ref) < REL_L2


def test_ffn_wider_than_64kb_of_lds(tmp_path):
    """An FFN 20480 wide: the down projection's input (80 KB as fp32) is staged in more than
    the 64 KB of LDS the matvec used to cap its input at; decode logits equal the oracle's
    step by step, and the prefill (GEMM K = 20480) equals the decode."""
    d = pyq35.default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                           attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=20480,
                           vocab_size=1024, native_max_context=4096)
    path = str(tmp_path / "wideffn")
    pyq35.synth_write_model(path, d, seed=4, std=0.02)
    prompt = pyq35.synth_token_ids(6, d.vocab_size, 24)
    m = pyq35.Model(path, 64)
    o = op.Oracle(path, 64)
    lg = np.stack([m.step(int(t))[0] for t in prompt])
    ref = np.stack([o.step(int(t)) for t in prompt])
    o.close()
    m.close()
    assert rel_l2(lg, ref) < REL_L2
    m = pyq35.Model(path, 64)
    pf = m.prefill(prompt)
    m.close()
    assert rel_l2(pf, lg) < REL_L2


def test_prefill_widths_not_multiple_of_32(tmp_path):
    """Hidden 264 and FFN 520 (multiples of 8, not of 32): the prefill keeps its activations
    row-major and the projections take the three-part bf16 GEMM; the prefill logits equal the
    oracle's step logits token by token."""
    d = pyq35.default_dims(hidden_size=264, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                           attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=520,
                           vocab_size=1024, native_max_context=4096)
    path = str(tmp_path / "odd")
    pyq35.synth_write_model(path, d, seed=7, std=0.02)
    prompt = pyq35.synth_token_ids(7, d.vocab_size, 40)
    m = pyq35.Model(path, 64)
    pf = m.prefill(prompt)
    m.close()
    o = op.Oracle(path, 64)
    ref = np.stack([o.step(int(t)) for t in prompt])
    o.close()
    assert rel_l2(pf, ref) < REL_L2


def test_decode_hidden_staged_through_lds(tmp_path):
    """Hidden 2560 (not a width whose input the matvec keeps in registers): the first
    projection reads the token's embedding row through the LDS-staged prologue and stores it
    as the residual stream; decode logits equal the oracle's step by step, and the device
    greedy loop equals the step-by-step argmax."""
    d = pyq35.default_dims(hidden_size=2560, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                           attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=512,
                           vocab_size=1024, native_max_context=4096)
    path = str(tmp_path / "h2560")
    pyq35.synth_write_model(path, d, seed=11, std=0.02)
    prompt = pyq35.synth_token_ids(12, d.vocab_size, 12)
    m = pyq35.Model(path, 64)
    o = op.Oracle(path, 64)
    lg = np.stack([m.step(int(t))[0] for t in prompt])
    ref = np.stack([o.step(int(t)) for t in prompt])
    assert rel_l2(lg, ref) < REL_L2
    tok = int(np.argmax(lg[-1]))
    ids = m.decode_greedy(tok, 6)
    want = []
    for _ in range(6):
        tok = int(np.argmax(o.step(tok)))
        want.append(tok)
    o.close()
    m.close()
    np.testing.assert_array_equal(ids, want)


def _set_all_embedding_rows_to_row0(path: str) -> None:
    """Rewrites the checkpoint's embedding (the tied output head) with every row a copy of
    row 0, in place (safetensors: 8-byte header length, JSON header, raw data)."""
    f = os.path.join(path, "model.safetensors")
    with open(f, "r+b") as fh:
        n = int.from_bytes(fh.read(8), "little")
        hdr = json.loads(fh.read(n))
        name = next(k for k in hdr if k.endswith("embed_tokens.weight"))
        t = hdr[name]
        rows, cols = t["shape"]
        b0, b1 = t["data_offsets"]
        assert t["dtype"] == "BF16" and b1 - b0 == rows * cols * 2
        fh.seek(8 + n + b0)
        row0 = fh.read(cols * 2)
        fh.seek(8 + n + b0)
        fh.write(row0 * rows)


def test_greedy_ties_take_the_first_index(tmp_path):
    """Every row of the tied embedding / output head equal, so every logit of a step is the
    same value: the greedy id is the first index, 0 (the reference's first-maximum rule),
    through the output head's per-workgroup argmax partials (40000 rows: 2048 workgroups of
    several row groups each) and the final pass."""
    d = pyq35.default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                           attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=512,
                           vocab_size=40000, native_max_context=4096)
    path = str(tmp_path / "ties")
    pyq35.synth_write_model(path, d, seed=13, std=0.02)
    _set_all_embedding_rows_to_row0(path)
    m = pyq35.Model(path, 64)
    lg, am = m.step(123)
    assert np.all(lg == lg[0]) and am == 0
    ids = m.decode_greedy(7, 5)
    m.close()
    np.testing.assert_array_equal(ids, np.zeros(5, np.int32))
