"""Writes the golden fixtures of tests/golden/ from the reference engine.

The reference (Qwen3.5-CPU-cpp) is compiled from its own sources by oracle/Makefile into
oracle/_ref/libq35ref.so; this script drives it through oracle/ref_harness.cpp on
synthetic checkpoints made by q35_synth_write_model and stores small input/output vectors:

  tiny.npz       tiny shape: checkpoint sha256, prompt, logits of every prompt step,
                 residual stream after every layer of every prompt step (from runs of the
                 reference truncated to 1..L layers), 16 greedy ids, GDN state / conv window /
                 K,V rows after 512 steps, and single-mixer cases with injected state
  tiny_gqa.npz   the same for a shape with v_heads = 2 k_heads and GQA group 4 (decode only)
  untied_prefill.npz  the reference's QwenForward::prefill logits of the tiny shape with a
                 separate lm_head: its output head is the embedding (src/qwen_forward.cpp:193-199),
                 not the lm_head the step uses, over all the embedding's rows
  c1_08b.npz     0.8B shape: checkpoint sha256, prompt, 128 greedy ids,
                 top logits and per-layer residuals at three positions

Run from the repository root: python tests/golden/make_golden.py [--skip-08b]
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "qwen3.5-cpu-cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle_py as op  # noqa: E402
import pyq35  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for blk in iter(lambda: f.read(1 << 24), b""):
            h.update(blk)
    return h.hexdigest()


def per_layer_trace(model_dir, ids, n_layers, max_ctx, record):
    """Residual stream after layer l at each recorded step, from reference runs truncated
    to l+1 layers: returns [len(record)][n_layers][H]."""
    out = None
    for l in range(n_layers):
        r = op.Ref(model_dir, max_ctx, l + 1)
        for t, tok in enumerate(ids):
            r.step(int(tok))
            if t in record:
                h = r.hidden()
                if out is None:
                    out = np.zeros((len(record), n_layers, h.size), np.float32)
                out[record.index(t), l] = h
        r.close()
    return out


def mixer_cases(model_dir, dims, seed):
    """Single-mixer calls of the reference on injected inputs/state: one GDN layer (0)
    and one attention layer (attn_interval - 1)."""
    lib = op.Ref.lib()
    d = dims
    H = d.hidden_size
    conv = 2 * d.gdn_k_heads * 128 + d.gdn_v_heads * 128
    out = {}
    max_ctx = 300
    r = op.Ref(model_dir, max_ctx)
    rng = np.random.default_rng(seed)
    # GDN layer 0 at position 7 with a random state and window
    normed = rng.standard_normal(H).astype(np.float32)
    S0 = (0.1 * rng.standard_normal((d.gdn_v_heads, 128, 128))).astype(np.float32)
    W0 = rng.standard_normal((conv, 3)).astype(np.float32)
    op.view(lib.ref_normed(r.h), (H,))[:] = normed
    op.view(lib.ref_gdn_state(r.h, 0), S0.shape)[:] = S0
    op.view(lib.ref_conv_state(r.h, 0), W0.shape)[:] = W0
    lib.ref_set_position(r.h, 7)
    mix = np.zeros(H, np.float32)
    lib.ref_mixer(r.h, 0, mix.ctypes.data)
    out.update(gdn_in=normed, gdn_S0=S0, gdn_W0=W0, gdn_out=mix,
               gdn_S1=op.view(lib.ref_gdn_state(r.h, 0), S0.shape).copy(),
               gdn_W1=op.view(lib.ref_conv_state(r.h, 0), W0.shape).copy())
    # attention layer at position 64 over a random cache (65 positions: two full 32-row
    # sub-chunks and a one-row remainder in the split-K kernel)
    al = d.attn_interval - 1
    pos = 64
    normed = rng.standard_normal(H).astype(np.float32)
    kv_shape = (max_ctx, d.attn_kv_heads, 256)
    K0 = np.zeros(kv_shape, np.float32)
    V0 = np.zeros(kv_shape, np.float32)
    K0[:pos] = rng.standard_normal((pos, d.attn_kv_heads, 256))
    V0[:pos] = rng.standard_normal((pos, d.attn_kv_heads, 256))
    op.view(lib.ref_normed(r.h), (H,))[:] = normed
    op.view(lib.ref_kcache(r.h, 0), kv_shape)[:] = K0
    op.view(lib.ref_vcache(r.h, 0), kv_shape)[:] = V0
    lib.ref_set_position(r.h, pos)
    mix = np.zeros(H, np.float32)
    lib.ref_mixer(r.h, al, mix.ctypes.data)
    out.update(attn_in=normed, attn_K0=K0[:pos], attn_V0=V0[:pos], attn_out=mix,
               attn_krow=op.view(lib.ref_kcache(r.h, 0), kv_shape)[pos].copy(),
               attn_vrow=op.view(lib.ref_vcache(r.h, 0), kv_shape)[pos].copy())
    r.close()
    return out


def tiny_fixture(name: str, prefill: bool):
    dims = pyq35.dims_for(name)
    with tempfile.TemporaryDirectory() as tmp:
        mdir = os.path.join(tmp, name)
        pyq35.synth_write_model(mdir, dims, seed=0, std=0.02)
        digest = sha256(os.path.join(mdir, "model.safetensors"))
        prompt = pyq35.synth_token_ids(1, dims.vocab_size, 16)
        n = len(prompt)
        r = op.Ref(mdir, 600)
        logits = np.stack([r.step(int(t)) for t in prompt])
        r.close()
        trace = per_layer_trace(mdir, prompt, dims.n_layers_total, 600, list(range(n)))
        r = op.Ref(mdir, 600)
        greedy = r.generate_greedy(prompt, 16)
        r.close()
        # 512 steps on a seeded token stream: GDN state, conv window and K/V rows
        long_ids = pyq35.synth_token_ids(3, dims.vocab_size, 512)
        r = op.Ref(mdir, 600)
        for t in long_ids:
            lg512 = r.step(int(t))
        lib = op.Ref.lib()
        conv = 2 * dims.gdn_k_heads * 128 + dims.gdn_v_heads * 128
        S512 = op.view(lib.ref_gdn_state(r.h, 0), (dims.gdn_v_heads, 128, 128)).copy()
        W512 = op.view(lib.ref_conv_state(r.h, 0), (conv, 3)).copy()
        K512 = op.view(lib.ref_kcache(r.h, 0), (600, dims.attn_kv_heads, 256))[:512].copy()
        V512 = op.view(lib.ref_vcache(r.h, 0), (600, dims.attn_kv_heads, 256))[:512].copy()
        h512 = r.hidden()
        r.close()
        fx = dict(sha256=np.array(digest), prompt=prompt, logits=logits, trace=trace,
                  greedy=greedy, long_ids=long_ids, S512=S512, W512=W512,
                  K512_last=K512[-8:], V512_last=V512[-8:], K512_sum=K512.sum(axis=(1, 2)),
                  V512_sum=V512.sum(axis=(1, 2)), logits512=lg512, hidden512=h512)
        fx.update(mixer_cases(mdir, dims, seed=5))
        if prefill:
            pr = np.zeros((n, dims.vocab_size), np.float32)
            r = op.Ref(mdir, 600)
            lib.ref_prefill(r.h, prompt.ctypes.data, n, pr.ctypes.data)
            r.close()
            fx["prefill_logits"] = pr
    np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **fx)
    print(f"{name}: sha256 {digest}, greedy {greedy.tolist()}")


def untied_prefill_fixture():
    dims = pyq35.dims_for("tiny_untied")
    with tempfile.TemporaryDirectory() as tmp:
        mdir = os.path.join(tmp, "tiny_untied")
        pyq35.synth_write_model(mdir, dims, seed=0, std=0.02)
        digest = sha256(os.path.join(mdir, "model.safetensors"))
        prompt = pyq35.synth_token_ids(1, dims.vocab_size, 16)
        n = len(prompt)
        r = op.Ref(mdir, 600)
        pr = r.prefill(prompt)
        step = np.stack([r.step(int(t)) for t in prompt])
        r.close()
    assert pr.shape == (n, dims.vocab_size)
    np.savez_compressed(os.path.join(OUT, "untied_prefill.npz"), sha256=np.array(digest), prompt=prompt,
                        prefill_logits=pr, step_logits=step)
    print(f"untied prefill: sha256 {digest}, rel distance of the two heads "
          f"{np.linalg.norm(pr - step) / np.linalg.norm(step):.3g}")


def c1_fixture(model_root: str):
    dims = pyq35.dims_for("0.8b")
    mdir = os.path.join(model_root, "q35_synth_0.8b_seed0")
    if not os.path.exists(os.path.join(mdir, "model.safetensors")):
        pyq35.synth_write_model(mdir, dims, seed=0, std=0.02)
    digest = sha256(os.path.join(mdir, "model.safetensors"))
    prompt = pyq35.synth_token_ids(1, dims.vocab_size, 32)
    n_new = 128
    max_ctx = len(prompt) + n_new + 2
    r = op.Ref(mdir, max_ctx)
    greedy = r.generate_greedy(prompt, n_new)
    r.close()
    seq = np.concatenate([prompt, greedy[:-1]])  # the tokens fed to step(), in order
    record = [0, len(prompt) - 1, len(seq) - 1]
    trace = per_layer_trace(mdir, seq, dims.n_layers_total, max_ctx, record)
    # logits at the recorded positions from the full model: top-16 and moments
    r = op.Ref(mdir, max_ctx)
    tops_i, tops_v, moments = [], [], []
    for t, tok in enumerate(seq):
        lg = r.step(int(tok))
        if t in record:
            idx = np.argsort(-lg, kind="stable")[:16]
            tops_i.append(idx.astype(np.int32))
            tops_v.append(lg[idx])
            moments.append([float(lg.astype(np.float64).sum()), float((lg.astype(np.float64) ** 2).sum())])
    r.close()
    np.savez_compressed(os.path.join(OUT, "c1_08b.npz"), sha256=np.array(digest), prompt=prompt,
                        greedy=greedy, record=np.array(record, np.int32), trace=trace,
                        top_idx=np.stack(tops_i), top_val=np.stack(tops_v),
                        moments=np.array(moments))
    print(f"0.8b: sha256 {digest}, greedy head {greedy[:16].tolist()}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-08b", action="store_true")
    ap.add_argument("--only", choices=["untied_prefill"], help="write one fixture only")
    ap.add_argument("--model-root", default=tempfile.gettempdir())
    a = ap.parse_args()
    if not op.ref_available():
        sys.exit("oracle/_ref/libq35ref.so missing: build it with make -C oracle (needs the reference tree)")
    if a.only == "untied_prefill":
        untied_prefill_fixture()
        return
    tiny_fixture("tiny", prefill=True)
    tiny_fixture("tiny_gqa", prefill=False)
    tiny_fixture("tiny_untied", prefill=False)
    untied_prefill_fixture()
    if not a.skip_08b:
        c1_fixture(a.model_root)


if __name__ == "__main__":
    main()
