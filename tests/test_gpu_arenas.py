"""The device memory plan and the prefill boundary: the prompt arena planned at creation
(reported in the budget, no allocation afterwards, larger blocks refused), the lazily made
one reused for smaller blocks, the KV capacity grown in place (q35_model_reserve_context,
weights kept) and planned from the device's memory by the memory equation
(src/memory_budget.cpp:56-81), the prefill's output head (QwenForward::prefill's embedding
rule, src/qwen_forward.cpp:193-199), and the QwenForward C++ drop-in driven from an
engine-side program."""
import os
import subprocess

import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import REL_L2, golden, rel_l2

pytestmark = pytest.mark.gpu
CPP = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp")


def allocs():
    return pyq35.lib.q35_device_alloc_count()


def rows_close(a, b):
    return max(rel_l2(a[t], b[t]) for t in range(len(a)))


def test_prompt_arena_planned_at_creation(model_dirs):
    g = golden("tiny")
    ids = np.asarray(g["long_ids"][:300], np.int32)
    lazy = pyq35.Model(model_dirs["tiny"], 600)
    lazy.set_prefill_block(128)
    ref = lazy.prefill(ids)
    lazy.close()
    m = pyq35.Model(model_dirs["tiny"], 600, prefill_block=256)
    b = m.budget()
    assert b["prompt_arena_bytes"] > 0
    n0 = allocs()
    out = m.prefill(ids)                       # blocks of the planned 256 tokens
    m.set_prefill_block(64)                    # a smaller block fits the planned arena
    out64 = m.prefill(ids)
    assert allocs() == n0
    assert rows_close(out, ref) < REL_L2 and rows_close(out64, ref) < REL_L2
    with pytest.raises(pyq35.Q35Error) as e:   # beyond the planned block
        m.set_prefill_block(512)
    assert e.value.status == -6
    assert m.budget() == b
    m.close()


def test_lazy_prompt_arena_reused_for_smaller_blocks(model_dirs):
    g = golden("tiny")
    ids = np.asarray(g["long_ids"][:200], np.int32)
    m = pyq35.Model(model_dirs["tiny"], 600)
    assert m.budget()["prompt_arena_bytes"] == 0
    m.set_prefill_block(256)
    n0 = allocs()
    m.prefill(ids, want_logits=False)
    assert allocs() == n0 + 1
    size = m.budget()["prompt_arena_bytes"]
    m.set_prefill_block(32)
    m.prefill(ids, want_logits=False)
    assert allocs() == n0 + 1 and m.budget()["prompt_arena_bytes"] == size
    m.set_prefill_block(512)
    m.prefill(ids, want_logits=False)
    assert allocs() == n0 + 2 and m.budget()["prompt_arena_bytes"] > size
    m.close()


def test_reserve_context_keeps_the_weights(model_dirs):
    g = golden("tiny")
    ids = np.asarray(g["long_ids"][:150], np.int32)
    m = pyq35.Model(model_dirs["tiny"], 64)
    with pytest.raises(pyq35.Q35Error):
        m.prefill(ids)
    n0 = allocs()
    w0 = m.budget()["weight_bytes"]
    m.reserve_context(200)
    assert allocs() == n0 + 2                  # the KV and scratch arenas only
    assert m.max_context == 200 and m.position == 0
    assert m.budget()["weight_bytes"] == w0
    assert m.budget()["kv_cache_bytes"] == 1 * 200 * 2 * 1 * 256 * 4
    lg = m.prefill(ids)
    ids2 = m.decode_greedy(int(np.argmax(lg[-1])), 8)
    m.reserve_context(100)                     # not larger: nothing changes
    assert m.max_context == 200 and allocs() == n0 + 3  # + the prompt arena of the prefill
    m.close()
    fresh = pyq35.Model(model_dirs["tiny"], 200)
    ref = fresh.prefill(ids)
    np.testing.assert_array_equal(fresh.decode_greedy(int(np.argmax(ref[-1])), 8), ids2)
    fresh.close()
    assert rows_close(lg, ref) < REL_L2


def test_failed_reserve_context_leaves_a_usable_model(model_dirs):
    """A context too large for the device (2^30 positions: terabytes of KV) is refused with
    the HIP status; the model keeps arenas of its old size (made again, zeroed, position 0)
    and decodes exactly as a fresh model of that size."""
    g = golden("tiny")
    ids = np.asarray(g["long_ids"][:40], np.int32)
    m = pyq35.Model(model_dirs["tiny"], 64)
    m.prefill(ids, want_logits=False)
    with pytest.raises(pyq35.Q35Error) as e:
        m.reserve_context(2**30)
    assert e.value.status == -2
    assert m.max_context == 64 and m.position == 0
    assert m.budget()["kv_cache_bytes"] == 1 * 64 * 2 * 1 * 256 * 4
    lg = m.prefill(ids)
    got = m.decode_greedy(int(np.argmax(lg[-1])), 8)
    m.close()
    fresh = pyq35.Model(model_dirs["tiny"], 64)
    ref = fresh.prefill(ids)
    np.testing.assert_array_equal(fresh.decode_greedy(int(np.argmax(ref[-1])), 8), got)
    fresh.close()
    assert rows_close(lg, ref) < REL_L2


def test_planned_block_beyond_max_context_then_reserve(model_dirs):
    """A block planned beyond max_context gets an arena for max_context tokens; after the
    context grows, prompts run in blocks of that size (no refusal, no new arena)."""
    g = golden("tiny")
    ids = np.asarray(g["long_ids"][:200], np.int32)
    m = pyq35.Model(model_dirs["tiny"], 48, prefill_block=256)
    m.reserve_context(256)
    n0 = allocs()
    out = m.prefill(ids)
    assert allocs() == n0
    m.close()
    lazy = pyq35.Model(model_dirs["tiny"], 256)
    lazy.set_prefill_block(48)
    ref = lazy.prefill(ids)
    lazy.close()
    assert rows_close(out, ref) < REL_L2


def test_max_context_planned_by_the_memory_equation(tmp_path):
    """max_context 0: the KV capacity comes from solve_max_context against the device's
    memory, capped at the native context (here 131072, the long-decode workload's cap: the
    equation alone would give millions of positions)."""
    d = pyq35.dims_for("2b")
    d.n_layers_total = 4
    d.vocab_size = 4096
    d.native_max_context = 131072
    path = str(tmp_path / "m")
    pyq35.synth_write_model(path, d, seed=1, std=0.02)
    m = pyq35.Model(path, 0)
    assert m.max_context == 131072
    b = m.budget()
    assert b["kv_cache_bytes"] == 1 * 131072 * 2 * 2 * 256 * 4
    # the equation itself, with the model's fixed costs, allows far more than the cap
    free, total = pyq35.Hip().mem_info()
    d.native_max_context = 2**31 - 1  # ModelConfig keeps the cap in an int
    uncapped = pyq35.lib.q35_solve_max_context(d, total, b["weight_bytes"], b["gdn_state_bytes"] + b["gdn_conv_bytes"],
                                               b["activation_bytes"], 0, 1 << 30, 4)
    assert uncapped > 131072
    # and the model runs at the far end of its context
    m.fill_synthetic(131072 - 4, seed=3)
    out = m.decode_greedy(1, 4)
    assert m.position == 131072 and len(out) == 4
    m.close()


def test_prefill_output_heads_vs_reference(model_dirs):
    """The untied checkpoint: the default prefill head is the step's (lm_head); the embedding
    head reproduces the reference's QwenForward::prefill logits."""
    g = golden("untied_prefill")
    m = pyq35.Model(model_dirs["tiny_untied"], 64)
    assert m.prefill_logits_width == 1024
    lg = m.prefill(g["prompt"])
    assert rows_close(lg, g["step_logits"]) < REL_L2
    m.set_prefill_head(True)
    lg = m.prefill(g["prompt"])
    assert rows_close(lg, g["prefill_logits"]) < REL_L2
    # decoding after the prefill still uses the step's head
    o = op.Oracle(model_dirs["tiny_untied"], 64)
    for t in g["prompt"]:
        ref = o.step(int(t))
    nxt = m.decode_greedy(int(np.argmax(ref)), 1)
    assert int(nxt[0]) == int(np.argmax(o.step(int(np.argmax(ref)))))
    o.close()
    m.close()


def test_qwen_forward_dropin_from_cpp(model_dirs, tmp_path):
    """An engine-side program on the QwenForward drop-in: the untied checkpoint's prefill
    logits equal the reference's (embedding head, rows of the embedding's width); a second,
    longer prompt (beyond the first device model's 4096 positions) grows the context without
    uploading the weights again, and its logits equal the oracle's prefill."""
    g = golden("untied_prefill")
    prompt2 = pyq35.synth_token_ids(9, 1024, 5000)
    out = str(tmp_path / "logits.f32")
    r = subprocess.run([os.path.join(CPP, "qwen_forward_caller"), model_dirs["tiny_untied"], out,
                        ",".join(str(int(t)) for t in g["prompt"]), ",".join(str(int(t)) for t in prompt2)],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [l for l in r.stdout.splitlines() if l.startswith("prompt")]
    n1 = int(lines[0].split("allocations ")[1])
    n2 = int(lines[1].split("allocations ")[1])
    assert n2 - n1 <= 3  # KV + scratch (+ a larger prompt arena): no second weight upload
    lg = np.fromfile(out, np.float32)
    first = lg[:16 * 1024].reshape(16, 1024)
    second = lg[16 * 1024:].reshape(5000, 1024)
    assert rows_close(first, g["prefill_logits"]) < REL_L2
    o = op.Oracle(model_dirs["tiny_untied"], 5008)
    ref = o.prefill(prompt2)
    o.close()
    errs = np.linalg.norm(second - ref, axis=1) / np.linalg.norm(ref, axis=1)
    print(f"5000-token prompt: worst row rel_l2 {errs.max():.3g}")
    assert errs.max() < REL_L2
