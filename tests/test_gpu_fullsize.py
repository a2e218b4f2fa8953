"""Parity at the configured sizes of the 2B-shaped workloads (hidden 2048, GDN 16 x 128,
attention 16 q / 2 kv heads x 256, rotary 64):

* the decode step at more than 8192 cached positions, run as the benchmark runs it (the
  captured step graph, the default 128-way split of the cache, the RoPE table, the GQA-8
  matrix-core attention kernel), against the oracle holding the same injected GDN state,
  conv window and K / V rows; fp32 and bf16 caches;
* a 4096-token prompt in one 4096-token block (the flash kernel's longest-first schedule,
  4096-row GEMMs, 64 chunks of the GDN state scan) against the oracle's sequential
  prefill (QwenForward::prefill, src/qwen_forward.cpp:154-206), per layer and token;
* the full 24-layer model over 4096 tokens: one 4096-token block, blocks of 256 and
  token-serial steps (QwenModel::step, src/qwen_model.cpp:211-239) each leave the state the
  oracle's sequential prefill leaves, and continue with its logits and greedy ids.

Bars: rel_l2 <= 1e-5 per layer / state / logits row, greedy ids identical.
A bf16 cache rounds appended rows to nearest even where the device's fp32 value can sit
within an ulp of a midpoint, so its logits and residuals are held to 2e-4 (the tolerance
of the bf16-cache model tests), its ids still identical."""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, rel_l2

pytestmark = pytest.mark.gpu

P_8K = 8192 + 37  # cached positions before the first step (not a multiple of any tile)


def rel_rows(a, b):
    """rel_l2 of each row of a against the same row of b (last axis)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b, axis=-1)
    return np.linalg.norm(a - b, axis=-1) / np.where(den > 0, den, 1.0)


@pytest.fixture(scope="module")
def m2b4(tmp_path_factory):
    """2B mixer shapes in a 4-layer model (3 GDN + 1 attention) with a 4096-token vocabulary."""
    d = pyq35.dims_for("2b")
    d.n_layers_total = 4
    d.vocab_size = 4096
    path = str(tmp_path_factory.mktemp("m2b4") / "model")
    pyq35.synth_write_model(path, d, seed=3, std=0.02)
    return path, d


def inject_state(m, o, d, P, kv_bf16, seed):
    """Same GDN states N(0, 0.1), conv windows N(0, 0.5) and K / V rows N(0, 1) for positions
    [0, P) in the device model and in the oracle; both at position P."""
    rng = np.random.default_rng(seed)
    n_gdn = d.n_layers_total - d.n_layers_total // d.attn_interval
    n_attn = d.n_layers_total // d.attn_interval
    conv = 2 * d.gdn_k_heads * 128 + d.gdn_v_heads * 128
    m.set_position(P)
    o.set_position(P)
    for i in range(n_gdn):
        S = (0.1 * rng.standard_normal((d.gdn_v_heads, 128, 128))).astype(np.float32)
        W = (0.5 * rng.standard_normal((conv, 3))).astype(np.float32)
        m.set_gdn_state(i, S)
        m.set_conv_state(i, W)
        o.gdn_state(i)[:] = S
        o.conv_state(i)[:] = W
    for l in range(n_attn):
        K = rng.standard_normal((P, d.attn_kv_heads, 256)).astype(np.float32)
        V = rng.standard_normal((P, d.attn_kv_heads, 256)).astype(np.float32)
        if kv_bf16:  # the cache holds these rows rounded to nearest even
            K, V = op.round_bf16(K), op.round_bf16(V)
        m.set_kv(l, 0, K, V)
        o.kcache(l)[:P] = K
        o.vcache(l)[:P] = V


@pytest.mark.parametrize("kv", ["fp32", "bf16"])
def test_decode_2b_after_8k_positions_through_graph(m2b4, kv):
    path, d = m2b4
    bf16 = kv == "bf16"
    max_ctx = P_8K + 16
    m = pyq35.Model(path, max_ctx, kv_bytes_per_elem=2 if bf16 else 4)
    o = op.Oracle(path, max_ctx, kv_bf16=bf16)
    try:
        decode_parity(m, o, d, P_8K, kv)
    finally:
        m.close()
        o.close()


@pytest.fixture(scope="module")
def m2b4_131k(tmp_path_factory):
    """The 4-layer 2B-shaped model with a native context of 131072 (the long-decode cap)."""
    d = pyq35.dims_for("2b")
    d.n_layers_total = 4
    d.vocab_size = 4096
    d.native_max_context = 131072
    path = str(tmp_path_factory.mktemp("m2b4_131k") / "model")
    pyq35.synth_write_model(path, d, seed=4, std=0.02)
    return path, d


@pytest.mark.timeout(900)
@pytest.mark.parametrize("kv", ["fp32", "bf16"])
def test_decode_2b_at_131k_context_planned_by_memory_equation(m2b4_131k, kv):
    """The long-context decode as the long-decode workload runs it: max_context 0, so the KV
    arena is planned by solve_max_context (src/memory_budget.cpp:56-81) and capped at 131072;
    the default split count for that arena, the RoPE table rows past 131000 (angles in double,
    src/forward_pass.cpp:102-112), the captured step graph and the greedy run, against the
    oracle holding the same state with 131060 cached positions (src/qwen_model.cpp:106-152)."""
    path, d = m2b4_131k
    bf16 = kv == "bf16"
    m = pyq35.Model(path, 0, kv_bytes_per_elem=2 if bf16 else 4)
    assert m.max_context == 131072
    o = op.Oracle(path, 131072, kv_bf16=bf16)
    try:
        decode_parity(m, o, d, 131060, kv)
    finally:
        m.close()
        o.close()


def decode_parity(m, o, d, P, kv):
    """Inject the same state with P cached positions into the device model and the oracle,
    then compare graph-replayed steps, a greedy run, one layer-traced step and the appended
    cache rows."""
    bf16 = kv == "bf16"
    tol = REL_L2 if not bf16 else 2e-4
    inject_state(m, o, d, P, bf16, seed=11)
    ids = pyq35.synth_token_ids(5, d.vocab_size, 6)
    worst = 0.0
    # graph-replayed steps (layer trace and timing off): logits, argmax, residual
    for t in ids:
        lg, am = m.step(int(t))
        ref = o.step(int(t))
        e = rel_l2(lg, ref)
        worst = max(worst, e)
        assert e < tol, f"logits at position {o.position - 1}: {e}"
        assert am == int(np.argmax(ref))
        assert rel_l2(m.hidden(), o.hidden()) < tol
    # greedy decoding with no host round trip between the steps
    first = int(np.argmax(ref))
    got = m.decode_greedy(first, 4)
    want, tok = [], first
    for _ in range(4):
        tok = int(np.argmax(o.step(tok)))
        want.append(tok)
    np.testing.assert_array_equal(got, want)
    # one more step with the per-layer trace (eager launches) against the oracle's trace
    rtr = o.enable_trace(rows=1)
    m.set_layer_trace(True)
    lg, _ = m.step(int(want[-1]))
    ref = o.step(int(want[-1]))
    tr = m.layer_trace()
    errs = rel_rows(tr, rtr[0])
    print(f"{kv} at {P} positions: worst logits rel_l2 {worst:.3g}, per-layer {errs.max():.3g}")
    assert errs.max() < tol
    assert rel_l2(lg, ref) < tol
    # the cache rows the steps appended
    n_new = len(ids) + 4 + 1
    for l in range(d.n_layers_total // d.attn_interval):
        K, V = m.kv(l, P, n_new)
        assert rel_l2(K, o.kcache(l)[P:P + n_new]) < tol
        assert rel_l2(V, o.vcache(l)[P:P + n_new]) < tol


@pytest.mark.timeout(900)
def test_prefill_4096_tokens_in_one_block_vs_oracle(m2b4):
    path, d = m2b4
    T = 4096
    ids = pyq35.synth_token_ids(2, d.vocab_size, T)
    m = pyq35.Model(path, T + 8)
    m.set_prefill_block(T)
    lg, tr = m.extend(ids, want_logits=True, want_trace=True)
    m.close()
    o = op.Oracle(path, T + 8)
    rtr = o.enable_trace(rows=T)
    ref = o.prefill(ids)
    o.close()
    errs = rel_rows(tr, rtr)  # [T][layers]
    t_bad, l_bad = np.unravel_index(int(np.argmax(errs)), errs.shape)
    print(f"4096-token block: worst per-layer rel_l2 {errs.max():.3g} (token {t_bad}, layer {l_bad}), "
          f"worst logits row {rel_rows(lg, ref).max():.3g}")
    assert errs.max() < REL_L2
    assert rel_rows(lg, ref).max() < REL_L2
    np.testing.assert_array_equal(np.argmax(lg, axis=1), np.argmax(ref, axis=1))


def snapshot(m, d, n):
    n_gdn = d.n_layers_total - d.n_layers_total // d.attn_interval
    n_attn = d.n_layers_total // d.attn_interval
    kv = [m.kv(l, 0, n) for l in range(n_attn)]
    return {
        "S": [m.gdn_state(i) for i in range(n_gdn)],
        "W": [m.conv_state(i) for i in range(n_gdn)],
        "K": [k for k, _ in kv],
        "V": [v for _, v in kv],
        "hidden": m.hidden(),
    }


def oracle_snapshot(o, d, n):
    n_gdn = d.n_layers_total - d.n_layers_total // d.attn_interval
    n_attn = d.n_layers_total // d.attn_interval
    return {
        "S": [o.gdn_state(i).copy() for i in range(n_gdn)],
        "W": [o.conv_state(i).copy() for i in range(n_gdn)],
        "K": [o.kcache(l)[:n].copy() for l in range(n_attn)],
        "V": [o.vcache(l)[:n].copy() for l in range(n_attn)],
        "hidden": o.hidden(),
    }


def state_errors(a, b):
    return {k: [rel_l2(x, y) for x, y in zip(a[k], b[k])] for k in ("S", "W", "K", "V")} | {
        "hidden": [rel_l2(a["hidden"], b["hidden"])]}


@pytest.mark.timeout(900)
def test_prefill_4096_tokens_24_layers_blocks_and_handoff(tmp_path_factory):
    """The full 2B-shaped model (24 layers, vocabulary 151936): 4095 prompt tokens prefilled
    in one block, in blocks of 256, and stepped one token at a time; each leaves the state
    (18 GDN states and conv windows, 6 layers of K / V rows, the residual) that the oracle's
    sequential prefill leaves (QwenForward::prefill's arithmetic, src/qwen_forward.cpp:83-152,
    with its final state kept -- the oracle's token-serial steps leave the same bits); the
    4096th token's step then gives the oracle's logits and greedy continuation."""
    d = pyq35.dims_for("2b")
    path = str(tmp_path_factory.mktemp("m2b24") / "model")
    pyq35.synth_write_model(path, d, seed=0, std=0.02)
    T = 4096
    ids = pyq35.synth_token_ids(2, d.vocab_size, T)
    m = pyq35.Model(path, T + 16)
    runs = {}
    try:
        for how in ("block4096", "block256", "serial"):
            m.reset()
            if how == "serial":
                for t in ids[:-1]:
                    m.step(int(t), want_logits=False)
            else:
                m.set_prefill_block(4096 if how == "block4096" else 256)
                m.extend(ids[:-1], want_logits=False)
            assert m.position == T - 1
            snap = snapshot(m, d, T - 1)
            lg, am = m.step(int(ids[-1]))
            snap["logits"] = lg
            snap["greedy"] = np.concatenate([[am], m.decode_greedy(am, 8)])
            runs[how] = snap
    finally:
        m.close()
    o = op.Oracle(path, T + 16)
    o.set_prefill_handoff(True)
    o.prefill(ids[:-1], want_logits=False)
    assert o.position == T - 1
    ref = oracle_snapshot(o, d, T - 1)
    ref["logits"] = o.step(int(ids[-1]))
    tok, greedy = int(np.argmax(ref["logits"])), []
    greedy.append(tok)
    for _ in range(8):
        tok = int(np.argmax(o.step(tok)))
        greedy.append(tok)
    o.close()
    for how, r in runs.items():
        errs = state_errors(r, ref)
        worst = {k: max(v) for k, v in errs.items()}
        print(f"{how} vs oracle: worst {worst}; GDN state per layer {np.round(np.array(errs['S']) * 1e6, 2)} e-6; "
              f"last-token logits {rel_l2(r['logits'], ref['logits']):.3g}")
    for how, r in runs.items():
        errs = state_errors(r, ref)
        for k, v in errs.items():
            assert max(v) < REL_L2, f"{how}: {k} {max(v)} (layer {int(np.argmax(v))})"
        assert rel_l2(r["logits"], ref["logits"]) < REL_L2, how
        np.testing.assert_array_equal(r["greedy"], greedy)
    # block boundaries carry the state exactly
    assert max(max(v) for v in state_errors(runs["block256"], runs["block4096"]).values()) < REL_L2
