"""Decode throughput of the 2B-shaped Qwen3.5 hybrid model at 8k context on one MI355X, with
the HBM roofline of the token-mixer kernels and the reference CPU path timed beside it.

A step is one greedy decode token through all 24 layers (18 Gated-DeltaNet + 6 gated
attention over an 8192-position fp32 KV cache), the tied lm_head and the device argmax.
Weights are a random-init bf16 checkpoint (N(0, 0.02), seed 0) written by the library's
synthetic writer; the KV cache is N(0,1) and the GDN states N(0, 0.1) (synthetic prefilled
cache). Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3.5-cpu-cpp_amd"))

METRIC = "decode tok/s + mixer HBM GB/s (%peak), 2B-shaped @8k ctx, 1 MI355X"
HBM_PEAK_GBS = 8000.0
GDN_LAYER_BYTES = 2_384_640  # per token per GDN layer (state r/w, conv window r/w, conv w, inputs, output)


def gdn_step_kernel_bytes(d) -> int:
    """Bytes of the decode step's GDN mixer kernel per layer: the conv window runs in the
    in-projection's epilogue, so the kernel moves the state (read and written), the convolved
    q / k / v, b / a, A_log / dt_bias and the readout (2,130,176 B at the 2B shape)."""
    KH, VH = d.gdn_k_heads, d.gdn_v_heads
    return 4 * (2 * VH * 128 * 128 + (2 * KH + VH) * 128 + 4 * VH + VH * 128)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class stdout_to_stderr:
    """Points file descriptor 1 at stderr for the block: the reference engine prints its
    arena plan on stdout, and stdout carries only the JSON result line."""

    def __enter__(self):
        sys.stdout.flush()
        self.saved = os.dup(1)
        os.dup2(2, 1)

    def __exit__(self, *exc):
        sys.stdout.flush()
        os.dup2(self.saved, 1)
        os.close(self.saved)


def ensure_model(path: str, dims, pyq35) -> None:
    st = os.path.join(path, "model.safetensors")
    if os.path.exists(st) and os.path.exists(os.path.join(path, "config.json")):
        return
    t = time.time()
    pyq35.synth_write_model(path, dims, seed=0, std=0.02, threads=0)
    log(f"wrote synthetic checkpoint {path} in {time.time() - t:.1f} s")


def weight_bytes_per_step(d) -> int:
    H, I, V = d.hidden_size, d.ffn_intermediate, d.vocab_size
    KD, VD, VH = d.gdn_k_heads * 128, d.gdn_v_heads * 128, d.gdn_v_heads
    NQ, NKV, HD = d.attn_q_heads, d.attn_kv_heads, d.attn_head_dim
    gdn = ((2 * KD + VD) + VD + 2 * VH) * H + H * VD
    attn = (2 * NQ * HD + 2 * NKV * HD) * H + H * NQ * HD
    ffn = 3 * H * I
    return 2 * (d.n_layers_gdn * gdn + d.n_layers_attn * attn + d.n_layers_total * ffn + V * H)


def cpu_baseline(model_dir: str, dims, ctx: int, n_steps: int) -> dict:
    """The reference engine (oracle/_ref) when it was built, else the oracle port, on the
    same checkpoint with a synthetic cache of ctx positions; times n_steps decode steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py as op
    import pyq35

    d = dims
    conv = 2 * d.gdn_k_heads * 128 + d.gdn_v_heads * 128
    kind = "reference" if op.ref_available() else "port"
    max_ctx = ctx + n_steps + 2
    t_load = time.time()
    if kind == "reference":
        eng = op.Ref(model_dir, max_ctx)
        lib = op.Ref.lib()
        kc = lambda i: op.view(lib.ref_kcache(eng.h, i), (max_ctx, d.attn_kv_heads, 256))  # noqa: E731
        vc = lambda i: op.view(lib.ref_vcache(eng.h, i), (max_ctx, d.attn_kv_heads, 256))  # noqa: E731
        st = lambda i: op.view(lib.ref_gdn_state(eng.h, i), (d.gdn_v_heads, 128, 128))  # noqa: E731
        setpos = lambda p: lib.ref_set_position(eng.h, p)  # noqa: E731
        step = eng.step
    else:
        eng = op.Oracle(model_dir, max_ctx)
        kc, vc, st, setpos, step = eng.kcache, eng.vcache, eng.gdn_state, eng.set_position, eng.step
    n = ctx * d.attn_kv_heads * 256
    for i in range(d.n_layers_attn):
        kc(i)[:ctx] = pyq35.synth_normal(n, 0, 1000 + i).reshape(ctx, d.attn_kv_heads, 256)
        vc(i)[:ctx] = pyq35.synth_normal(n, 0, 2000 + i).reshape(ctx, d.attn_kv_heads, 256)
    for i in range(d.n_layers_gdn):
        st(i)[:] = pyq35.synth_normal(d.gdn_v_heads * 128 * 128, 0, 3000 + i, 0.1).reshape(d.gdn_v_heads, 128, 128)
    setpos(ctx)
    log(f"cpu baseline ({kind}) loaded in {time.time() - t_load:.1f} s; timing {n_steps} steps")
    tok = 1
    step(tok)  # untimed warm-up step
    times = []
    for _ in range(n_steps):
        t0 = time.perf_counter()
        lg = step(tok)
        times.append(time.perf_counter() - t0)
        tok = int(np.argmax(lg))
    med = float(np.median(times))
    threads = op.threads()
    return {"value": 1.0 / med, "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"median of {n_steps} timed greedy decode steps of the same 2B-shaped checkpoint at "
                      f"positions {ctx + 2}..{ctx + n_steps + 1} (synthetic cache; {sum(times):.1f} s in all, "
                      f"{min(times) * 1e3:.0f}-{max(times) * 1e3:.0f} ms per step), OpenMP threads={threads}"}


def cpu_greedy_baseline(model_dir: str, dims, prompt_len: int, n_steps: int) -> dict:
    """The reference (oracle/_ref when built, else the oracle port): the prompt, then n_steps
    greedy steps of the same checkpoint, timed over the greedy steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py as op
    import pyq35

    kind = "reference" if op.ref_available() else "port"
    prompt = pyq35.synth_token_ids(1, dims.vocab_size, prompt_len)
    eng = op.Ref(model_dir, prompt_len + n_steps + 2) if kind == "reference" else op.Oracle(model_dir, prompt_len + n_steps + 2)
    lg = None
    for t in prompt:
        lg = eng.step(int(t))
    tok = int(np.argmax(lg))
    times = []
    for _ in range(n_steps):
        t0 = time.perf_counter()
        tok = int(np.argmax(eng.step(tok)))
        times.append(time.perf_counter() - t0)
    eng.close()
    return {"value": 1.0 / float(np.median(times)), "unit": "tok/s", "cores": op.threads(), "kind": kind,
            "sample": f"median of {n_steps} timed greedy steps after the {prompt_len}-token prompt "
                      f"({sum(times):.1f} s in all)"}


def bench_gdn(a) -> dict:
    """Isolated GDN decode: 18 layers of 16 x 128 x 128 fp32 state in one launch per token,
    `steps` sequential tokens (q/k/v/z/a/b drawn N(0,1), A_log and dt_bias N(0,1), state
    N(0, 0.1)). With --rotate R, R independent state sets are visited round-robin so the
    working set exceeds the 256 MB Infinity Cache."""
    import pyq35

    hip = pyq35.Hip()
    L, KH, VH, D = 18, 16, 16, 128
    CONV, VD = 2 * KH * D + VH * D, VH * D
    R = max(1, a.rotate)
    P = 32  # distinct per-token input sets on the device, cycled
    rng_seed = 7

    def normal(n, stream, std=1.0):
        return pyq35.synth_normal(n, rng_seed, stream, std)

    qkv = hip.upload(normal(P * L * CONV, 1))
    z = hip.upload(normal(P * L * VD, 2))
    b = hip.upload(normal(P * L * VH, 3))
    av = hip.upload(normal(P * L * VH, 4))
    convw = hip.upload(normal(L * CONV * 4, 5, 0.5))
    alog = hip.upload(normal(L * VH, 6))
    dtb = hip.upload(normal(L * VH, 7))
    normw = hip.upload(np.ones(L * D, np.float32))
    states = [hip.upload(normal(L * VH * D * D, 100 + r, 0.1)) for r in range(R)]
    rings = [hip.upload(np.zeros(L * 4 * CONV, np.float32)) for r in range(R)]
    out = hip.malloc(L * VD * 4)
    res = {}
    for fused in (False, True):
        def launch(t):
            r = t % R
            p = t % P
            args = pyq35.GdnDecodeArgs(
                n_layers=L, k_heads=KH, v_heads=VH, head_dim_k=D, head_dim_v=D, conv_kernel=4,
                pos=t // R, eps=1e-6, qkv=qkv + p * L * CONV * 4, z=z + p * L * VD * 4,
                b=b + p * L * VH * 4, a=av + p * L * VH * 4, conv_w=convw, A_log=alog,
                dt_bias=dtb, norm_w=normw if fused else None, conv_ring=rings[r],
                state=states[r], out=out)
            pyq35.check(pyq35.lib.q35_gdn_decode(args, None))
        for t in range(a.warmup):
            launch(t)
        hip.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0)
        for t in range(a.steps):
            launch(a.warmup + t)
        hip.record(e1)
        ms = hip.elapsed_ms(e0, e1)
        per = ms / a.steps
        nbytes = L * (GDN_LAYER_BYTES - (0 if fused else VD * 4))
        res["fused_norm" if fused else "split"] = {
            "us_per_token": per * 1e3, "tok_per_s": 1e3 / per, "GBs": nbytes / (per / 1e3) / 1e9,
            "frac": nbytes / (per / 1e3) / 1e9 / HBM_PEAK_GBS, "bytes_per_launch": nbytes}
    best = max(res.values(), key=lambda v: v["GBs"])
    return {"metric": "isolated GDN decode (18 layers x 16 heads of 128x128 fp32 state) tok/s",
            "value": best["tok_per_s"], "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": best["us_per_token"] / 1e3, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic N(0,1) inputs",
            "config": {"workload": "isolated GDN decode", "layers": L, "heads": VH, "state": "128x128",
                       "rotated_state_sets": R, "working_set_MiB": R * L * VH * D * D * 4 / 2**20},
            "roofline": {"bound": "hbm", "kernel": "gdn_decode (18 layers per launch)",
                         "achieved": best["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": best["frac"], "traffic": None, "bytes_per_launch": best["bytes_per_launch"],
                         "avg_launch_us": best["us_per_token"]},
            "variants": res}


def bench_attn(a) -> dict:
    """Isolated gated-attention decode at the 2B shape: 6 layers with their own fp32 KV
    caches (N(0,1)) at each context of --ctx-list, one new token per step across the 6 layers
    (q/k norm + RoPE + append + split-K softmax + gate). --kv bf16: bf16 caches. With
    --rotate R, up to R independent sets of the 6 caches are visited round-robin (as many as
    keep the working set near 1 GiB), so that the caches are read from HBM rather than from
    the 256 MB Infinity Cache."""
    import pyq35

    hip = pyq35.Hip()
    NQ, NKV, HD, L = 16, 2, 256, 6
    E = 2 if a.kv == "bf16" else 4

    def cache(n, stream):
        x = pyq35.synth_normal(n, 11, stream)
        if E == 2:  # nearest-even bf16 bit patterns
            u = x.view(np.uint32).astype(np.uint64)
            x = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return hip.upload(x)
    res = {}
    for ctx in a.ctx_list:
        maxc = ctx + 2 * (a.warmup + a.steps) + 1
        n = NKV * maxc * HD  # one layer's K (or V) cache
        set_bytes = 2 * L * n * E
        R = max(1, min(a.rotate, -(-(1 << 30) // set_bytes)))
        Ks = [cache(L * n, 2 * r) for r in range(R)]
        Vs = [cache(L * n, 2 * r + 1) for r in range(R)]
        qg = hip.upload(pyq35.synth_normal(L * 2 * NQ * HD, 12, 0))
        kn = hip.upload(pyq35.synth_normal(L * NKV * HD, 12, 1))
        vn = hip.upload(pyq35.synth_normal(L * NKV * HD, 12, 2))
        w = hip.upload(np.zeros(L * HD, np.float32))
        out = hip.malloc(L * NQ * HD * 4)
        row = {"kv_working_set_MiB": R * set_bytes / 2**20, "kv_sets": R}
        p = ctx
        for mode in ("batched", "per_layer"):
            args = pyq35.AttnDecodeArgs(q_heads=NQ, kv_heads=NKV, head_dim=HD, rotary_dim=64, pos=ctx,
                                        n_splits=a.attn_splits, n_layers=L if mode == "batched" else 1,
                                        max_context=maxc, rope_theta=1e7, eps=1e-6, kv_dtype=int(E == 2))
            ws = pyq35.lib.q35_attn_decode_workspace_bytes(args)
            wsp = hip.malloc(ws)
            args.out, args.workspace, args.workspace_bytes = out, wsp, ws

            def step(pos):
                args.pos = pos
                K, V = Ks[pos % R], Vs[pos % R]
                if mode == "batched":
                    args.qg, args.k_new, args.v_new, args.q_norm, args.k_norm = qg, kn, vn, w, w
                    args.k_cache, args.v_cache = K, V
                    pyq35.check(pyq35.lib.q35_attn_decode(args, None))
                else:
                    for l in range(L):
                        args.qg, args.k_new = qg + l * 2 * NQ * HD * 4, kn + l * NKV * HD * 4
                        args.v_new, args.q_norm, args.k_norm = vn + l * NKV * HD * 4, w, w
                        args.k_cache, args.v_cache = K + l * n * E, V + l * n * E
                        pyq35.check(pyq35.lib.q35_attn_decode(args, None))
            for _ in range(a.warmup):
                step(p)
                p += 1
            hip.sync()
            e0, e1 = hip.event(), hip.event()
            p_first = p
            hip.record(e0)
            for _ in range(a.steps):
                step(p)
                p += 1
            hip.record(e1)
            per = hip.elapsed_ms(e0, e1) / a.steps
            T = p_first + (a.steps + 1) / 2.0
            nbytes = L * (2 * NKV * HD * E * T + 59_392)
            row[mode] = {"ms_per_token": per, "GBs": nbytes / (per / 1e3) / 1e9,
                         "frac": nbytes / (per / 1e3) / 1e9 / HBM_PEAK_GBS}
            hip.free(wsp)
        res[str(ctx)] = row
        for q in Ks + Vs + [qg, kn, vn, w, out]:
            hip.free(q)
    key = str(8192) if "8192" in res else list(res)[0]
    r = res[key]["batched"]
    return {"metric": "isolated gated-attention decode (6 layers, 2B shape) mixer GB/s", "value": r["GBs"],
            "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": r["ms_per_token"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
            "data": "synthetic N(0,1) KV cache and inputs",
            "config": {"workload": "isolated attention decode", "context": int(key), "layers": L,
                       "heads": f"{NQ}q/{NKV}kv x {HD}", "kv_cache": a.kv,
                       "kv_sets": res[key]["kv_sets"], "kv_working_set_MiB": res[key]["kv_working_set_MiB"]},
            "roofline": {"bound": "hbm", "kernel": "attention decode (split-K + combine), 6 layers",
                         "achieved": r["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": r["frac"],
                         "traffic": None},
            "contexts": res}


FP32_MFMA_PEAK_TFS = 157.3
BF16_MFMA_PEAK_TFS = 2500.0
FP16_MFMA_PEAK_TFS = 2500.0
GDN_CHUNK_FLOPS = 5 * 64 * 64 * 128 * 2 + 3 * 64 * 128 * 128 * 2 + 64 ** 3 // 3 * 2 + 128 * 128


def projection_params(d) -> int:
    """Weights multiplied per token by the prefill GEMMs (every layer matrix, no lm_head)."""
    H, I = d.hidden_size, d.ffn_intermediate
    KD, VD, VH = d.gdn_k_heads * 128, d.gdn_v_heads * 128, d.gdn_v_heads
    NQ, NKV, HD = d.attn_q_heads, d.attn_kv_heads, d.attn_head_dim
    gdn = ((2 * KD + VD) + VD + 2 * VH) * H + H * VD
    attn = (2 * NQ * HD + 2 * NKV * HD) * H + H * NQ * HD
    return d.n_layers_gdn * gdn + d.n_layers_attn * attn + d.n_layers_total * 3 * H * I


def bench_prefill(a) -> dict:
    """Whole-prompt prefill of a 4096-token prompt (ids uniform, seed 2) at the 2B shape:
    the chunked GDN, the flash attention and the projection GEMMs of all 24 layers; the
    last row's logits and argmax (what decoding continues from), not every row's logits."""
    import pyq35

    d = pyq35.dims_for("2b")
    a.model_dir = a.model_dir or "/tmp/q35_synth_2b_seed0"
    ensure_model(a.model_dir, d, pyq35)
    T = a.prompt
    ids = pyq35.synth_token_ids(2, d.vocab_size, T)
    m = pyq35.Model(a.model_dir, T + 8, prefill_exact=a.prefill_exact)
    if a.prefill_block:
        m.set_prefill_block(a.prefill_block)
    for _ in range(max(1, a.warmup)):
        m.prefill(ids, want_logits=False)
    walls = []
    for _ in range(a.steps):
        pyq35.check(pyq35.lib.q35_model_synchronize(m.h))
        t0 = time.perf_counter()
        m.prefill(ids, want_logits=False)
        walls.append(time.perf_counter() - t0)
    wall = float(np.median(walls))
    m.set_kernel_timing(True)
    m.prefill(ids, want_logits=False)
    kt = m.kernel_times()
    m.set_kernel_timing(False)
    m.close()
    NQ, HD = d.attn_q_heads, d.attn_head_dim
    attn_flops = 4 * NQ * HD * T * (T + 1) / 2  # per layer, causal half
    nchunk = (T + 63) // 64
    gdn_flops = GDN_CHUNK_FLOPS * d.gdn_v_heads * nchunk  # per layer
    gemm_flops = 2.0 * T * projection_params(d)
    ms = {k: v[0] for k, v in kt.items()}
    n = {k: v[1] for k, v in kt.items()}
    # launches are per (block, layer); the flop counts above are per layer over the prompt
    attn_tfs = attn_flops * d.n_layers_attn / (ms["attn_prefill"] / 1e3) / 1e12
    gdn_tfs = gdn_flops * d.n_layers_gdn / (ms["gdn_prefill"] / 1e3) / 1e12
    gemm_tfs = gemm_flops / (ms["gemm"] / 1e3) / 1e12
    kernels = {k: {"ms": v[0], "launches": v[1]} for k, v in kt.items() if v[1]}
    dominant = max(("gemm", "attn_prefill", "gdn_prefill"), key=lambda k: ms[k])
    ach = {"gemm": gemm_tfs, "attn_prefill": attn_tfs, "gdn_prefill": gdn_tfs}[dominant]
    # The prefill's projection GEMM runs each fp32 product as two fp16 products (row-scaled
    # two-part activations, fp16 weight copies) on the 16-bit matrix cores, so its ceiling is
    # the dense fp16 peak over 2 in fp32-product terms; the flash attention as six bf16 part
    # products (peak / 6); the chunked GDN on the fp32 matrix cores.
    # (--prefill-exact: three exact bf16 parts, bf16 peak / 3)
    gemm_peak = BF16_MFMA_PEAK_TFS / 3 if a.prefill_exact else FP16_MFMA_PEAK_TFS / 2
    peaks = {"gemm": gemm_peak, "attn_prefill": BF16_MFMA_PEAK_TFS / 6, "gdn_prefill": FP32_MFMA_PEAK_TFS}
    peak = peaks[dominant]
    mixer_flops = d.n_layers_attn * attn_flops + d.n_layers_gdn * gdn_flops
    mixer_ms = ms["attn_prefill"] + ms["gdn_prefill"]
    res = {
        "metric": "prefill tok/s + MFMA TFLOP/s, 2B-shaped 4096-token prompt, 1 MI355X",
        "value": T / wall, "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": wall * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic: random-init bf16 weights N(0,0.02) seed 0, ids uniform seed 2",
        "config": {"workload": f"2B-shaped Qwen3.5 prefill of {T} tokens", "hidden": d.hidden_size,
                   "layers": "24 = 18 GDN + 6 gated attention", "prompt": T,
                   "block": a.prefill_block or min(4096, T + 8), "gdn_chunk": 64,
                   "gemm": ("three exact bf16 parts per fp32 activation" if a.prefill_exact else
                            "two row-scaled fp16 parts per fp32 activation, fp16 weight copies")},
        "roofline": {"bound": "mfma", "kernel": dominant, "achieved": ach, "peak": peak,
                     "unit": "TFLOP/s", "frac": ach / peak, "traffic": None,
                     "note": "fp32 flops of the algorithm; GEMM peak = dense fp16 MFMA peak / 2 (two "
                             "fp16 parts of each row-scaled fp32 activation against fp16 weight copies; "
                             "with --prefill-exact bf16 peak / 3, three exact bf16 parts); "
                             "flash attention = bf16 peak / 6 (six part products per fp32 product); GDN = "
                             "fp32 MFMA peak"},
        "mixers": {"attn_prefill_TFs": attn_tfs, "attn_prefill_frac": attn_tfs / peaks["attn_prefill"],
                   "gdn_prefill_frac": gdn_tfs / FP32_MFMA_PEAK_TFS,
                   "gdn_prefill_TFs": gdn_tfs, "gemm_TFs": gemm_tfs,
                   "mixer_TFs": mixer_flops / (mixer_ms / 1e3) / 1e12,
                   "mixer_ms": mixer_ms, "gemm_ms": ms["gemm"], "other_ms": ms["other"]},
        "kernels": kernels,
    }
    if not a.no_cpu_baseline:
        with stdout_to_stderr():
            res["cpu_baseline"] = cpu_prefill_baseline(a.model_dir, d, a.cpu_prompt)
    return res


def cpu_prefill_baseline(model_dir: str, dims, n_tok: int) -> dict:
    """QwenForward::prefill (oracle/_ref when built, else the oracle port) on the first
    n_tok ids of the same prompt."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_py as op
    import pyq35

    ids = pyq35.synth_token_ids(2, dims.vocab_size, n_tok)
    kind = "reference" if op.ref_available() else "port"
    r = op.Ref(model_dir, n_tok + 8) if kind == "reference" else op.Oracle(model_dir, n_tok + 8)
    r.prefill(ids[:1])  # first touch of every weight (the reference widens them once, cached)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        r.prefill(ids)
        times.append(time.perf_counter() - t0)
    r.close()
    dt = float(np.median(times))
    return {"value": n_tok / dt, "unit": "tok/s", "cores": op.threads(), "kind": kind,
            "sample": f"median of 5 prefills of the first {n_tok} prompt ids (every row's logits), "
                      f"{dt:.2f} s each"}


def calibration_copy(nbytes: int = 256 << 20) -> None:
    """One device-to-device copy of a known size (the runtime's copy kernel), the reference
    for scaling FETCH_SIZE / WRITE_SIZE counters to bytes in counter runs."""
    import pyq35

    hip = pyq35.Hip()
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.rt.hipMemcpy(pyq35.C.c_void_p(dst), pyq35.C.c_void_p(src), nbytes, 3)
    hip.sync()
    hip.free(src)
    hip.free(dst)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 64; 256 for --workload long)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--model", choices=["2b", "0.8b"], default="2b",
                    help="decode: 2B shape at --ctx (synthetic cache) or the 0.8B shape after a prompt")
    ap.add_argument("--model-dir", default="", help="checkpoint directory (written when absent)")
    ap.add_argument("--prompt-len", type=int, default=32, help="0.8b decode: prompt tokens")
    ap.add_argument("--cpu-steps", type=int, default=5, help="timed CPU steps (the median is reported)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=["decode", "long", "gdn", "attn", "prefill"], default="decode",
                    help="decode: full 2B-shaped decode step (default); long: 2B-shaped decode at the end of "
                         "a context planned by the memory equation (max_position_embeddings 131072); "
                         "gdn / attn: isolated mixers; prefill: 2B-shaped whole-prompt prefill")
    ap.add_argument("--prompt", type=int, default=4096, help="prefill: prompt tokens")
    ap.add_argument("--prefill-block", type=int, default=0, help="prefill: tokens per block (0 = auto)")
    ap.add_argument("--cpu-prompt", type=int, default=32, help="prefill: prompt tokens of the CPU sample")
    ap.add_argument("--rotate", type=int, default=1, help="gdn: independent state sets; attn: independent sets of the 6 KV caches "
                         "(as many as fit about 1 GiB), visited round-robin")
    ap.add_argument("--ctx-list", type=lambda s: [int(x) for x in s.split(",")], default=[2048, 8192, 32768])
    ap.add_argument("--attn-splits", type=int, default=0,
                    help="attention split-K count (0 = the library default)")
    ap.add_argument("--kv", choices=["fp32", "bf16"], default="fp32",
                    help="KV cache element type (decode, attn): fp32 is the reference's cache")
    ap.add_argument("--prefill-exact", action="store_true",
                    help="prefill: projection GEMMs on three exact bf16 parts (no fp16 weight copies)")
    ap.add_argument("--no-prefill-line", action="store_true",
                    help="default decode run: skip the 4096-token prefill measured beside it")
    ap.add_argument("--no-long-line", action="store_true",
                    help="default decode run: skip the 131072-context decode measured beside it")
    ap.add_argument("--no-mixer-lines", action="store_true",
                    help="default decode run: skip the isolated GDN / attention mixers measured beside it")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="finish with a 256 MiB device copy (reference for counter runs)")
    a = ap.parse_args()
    if a.steps is None:
        a.steps = 256 if a.workload == "long" else 64
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported "
              "(the multi-GPU sharding of the path is a design note, not built)", file=sys.stderr)
        sys.exit(2)
    if a.workload not in ("decode", "long"):
        result = {"gdn": bench_gdn, "attn": bench_attn, "prefill": bench_prefill}[a.workload](a)
        if a.calibration_copy:
            calibration_copy()
        print(json.dumps(result), flush=True)
        return
    print(json.dumps(bench_decode(a)), flush=True)


def bench_decode(a) -> dict:
    """The decode workloads: the 2B shape at --ctx positions of synthetic cache (default), the
    0.8B shape after a prompt (--model 0.8b), or the 2B shape at the end of a context the
    library plans itself (--workload long: KV arena sized by solve_max_context against the
    device's memory, capped by max_position_embeddings = 131072; the cache is filled up to
    the last warm-up + timed steps)."""
    import pyq35

    long_ctx = a.workload == "long"
    small = a.model == "0.8b" and not long_ctx
    d = pyq35.dims_for("0.8b" if small else "2b")
    if long_ctx:
        d.native_max_context = 131072
    model_dir = a.model_dir or ("/tmp/q35_synth_08b_seed0" if small else
                                "/tmp/q35_synth_2b_ctx131072_seed0" if long_ctx else "/tmp/q35_synth_2b_seed0")
    ensure_model(model_dir, d, pyq35)
    t = time.time()
    kv_elem = 2 if a.kv == "bf16" else 4
    if long_ctx:
        m = pyq35.Model(model_dir, 0, kv_bytes_per_elem=kv_elem)
        max_ctx = m.max_context
        ctx = max_ctx - a.warmup - 2 * a.steps - 1
    else:
        ctx = a.prompt_len if small else a.ctx
        max_ctx = ctx + a.warmup + 2 * a.steps + 4
        m = pyq35.Model(model_dir, max_ctx, kv_bytes_per_elem=kv_elem)
    log(f"model uploaded in {time.time() - t:.1f} s; max_context {max_ctx}; budget {m.budget()}")
    if a.attn_splits:
        m.set_attn_splits(a.attn_splits)
    hip = pyq35.Hip()
    if small:
        # the 0.8B-shaped greedy run: a prompt of uniform ids (seed 1) prefilled, then decode
        prompt = pyq35.synth_token_ids(1, d.vocab_size, ctx)
        lg = m.prefill(prompt)
        tok = int(np.argmax(lg[-1]))
    else:
        m.fill_synthetic(ctx, seed=0, state_std=0.1)
        tok = 1

    # warm-up (builds and replays the step graph)
    ids = m.decode_greedy(tok, a.warmup)
    tok = int(ids[-1])
    # timed: K greedy steps back to back on the device (graph replays), bracketed by syncs
    stream = pyq35.lib.q35_model_stream(m.h)
    e0, e1 = hip.event(), hip.event()
    pyq35.check(pyq35.lib.q35_model_synchronize(m.h))
    t0 = time.perf_counter()
    hip.record(e0, stream)
    ids = m.decode_greedy(tok, a.steps)
    hip.record(e1, stream)
    pyq35.check(pyq35.lib.q35_model_synchronize(m.h))
    wall = time.perf_counter() - t0
    dev_ms = hip.elapsed_ms(e0, e1)
    ms_per_step = 1e3 * wall / a.steps
    tok = int(ids[-1])
    log(f"{a.steps} steps: wall {wall * 1e3:.2f} ms, device {dev_ms:.2f} ms")

    # kernel-timed pass: the same steps launched eagerly with events around every launch
    p_first = m.position
    m.set_kernel_timing(True)
    m.decode_greedy(tok, a.steps)
    kt = m.kernel_times()
    m.set_kernel_timing(False)
    mean_n = p_first + (a.steps + 1) / 2.0  # mean attended positions (pos + 1) over the pass
    NKV, HD, NQ = d.attn_kv_heads, d.attn_head_dim, d.attn_q_heads
    attn_ms, attn_n = kt["attn_decode"]
    attn_avg_s = attn_ms / 1e3 / attn_n
    attn_bytes = 2 * NKV * HD * kv_elem * mean_n + NQ * HD * 4  # K and V rows + the queries
    attn_gbs = attn_bytes / attn_avg_s / 1e9
    mixer_ms = sum(kt[k][0] for k in ("attn_decode", "attn_combine"))
    mixer_bytes = 2 * NKV * HD * kv_elem * mean_n + 59_392  # per layer incl. projection outputs, append, output
    mixer_gbs = mixer_bytes * attn_n / (mixer_ms / 1e3) / 1e9
    gdn_ms, gdn_n = kt["gdn_decode"]
    gdn_gbs = gdn_step_kernel_bytes(d) * gdn_n / (gdn_ms / 1e3) / 1e9
    gemv_ms, gemv_n = kt["gemv"]
    wb = weight_bytes_per_step(d)
    gemv_gbs = wb * a.steps / (gemv_ms / 1e3) / 1e9
    kernels = {k: {"avg_us": 1e3 * v[0] / max(v[1], 1), "launches": v[1]} for k, v in kt.items()}

    result = {
        "metric": (METRIC if not (small or long_ctx) else
                   "decode tok/s, 0.8B-shaped greedy after a prompt, 1 MI355X" if small else
                   "decode tok/s + mixer HBM GB/s (%peak), 2B-shaped @131072 ctx (KV planned by "
                   "solve_max_context), 1 MI355X"),
        "value": a.steps / wall,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": ("synthetic: random-init bf16 weights N(0,0.02) seed 0, "
                 + (f"{ctx}-token prompt of uniform ids (seed 1) prefilled" if small
                    else "KV cache N(0,1), GDN state N(0,0.1)")),
        "config": {"workload": (f"{'0.8B' if small else '2B'}-shaped Qwen3.5 greedy decode at "
                                f"{'a ' + str(ctx) + '-token prompt' if small else str(ctx) + ' context'}"
                                + (f", KV arena of {max_ctx} positions planned by solve_max_context against "
                                   f"the device's memory" if long_ctx else "")),
                   "hidden": d.hidden_size, "layers": "24 = 18 GDN + 6 gated attention",
                   "gdn_heads": d.gdn_v_heads, "attn_heads": f"{NQ}q/{NKV}kv x {HD}",
                   "ffn": d.ffn_intermediate, "vocab": d.vocab_size, "context": ctx,
                   "batch": 1, "kv_cache": a.kv, "max_context": max_ctx},
        # the dominant kernel of the step by time: the bf16 matvec (every projection, the FFN
        # and the tied output head; 97 launches per step), bytes = the weights it streams
        "roofline": {"bound": "hbm", "kernel": "bf16 matvec (all projections + output head, per step)",
                     "achieved": gemv_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gemv_gbs / HBM_PEAK_GBS, "traffic": None,
                     "bytes_per_launch": wb / (gemv_n / a.steps), "avg_launch_us": 1e3 * gemv_ms / gemv_n},
        "roofline_attention": {"bound": "hbm", "kernel": "attention decode split-K partial (per layer)",
                               "achieved": attn_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": attn_gbs / HBM_PEAK_GBS, "traffic": None,
                               "bytes_per_launch": attn_bytes, "avg_launch_us": attn_avg_s * 1e6},
        "mixers": {
            "attention_mixer_GBs": mixer_gbs, "attention_mixer_frac": mixer_gbs / HBM_PEAK_GBS,
            "gdn_decode_GBs": gdn_gbs, "gdn_decode_frac": gdn_gbs / HBM_PEAK_GBS,
            "gemv_GBs": gemv_gbs, "gemv_frac": gemv_gbs / HBM_PEAK_GBS,
        },
        "kernels": kernels,
        "device_ms_per_step": dev_ms / a.steps,
    }
    m.close()
    if not (small or long_ctx) and not a.no_prefill_line:
        # the whole-prompt path measured in the same run (a 4096-token prefill of the same
        # checkpoint, 4 warm-up + 16 timed + 1 kernel-timed), so that its figures are timed by
        # whoever runs the default bench; `--workload prefill` gives the full line
        try:
            pa = argparse.Namespace(**vars(a))
            pa.steps, pa.warmup, pa.prompt, pa.prefill_block = 16, 4, 4096, 0
            pa.prefill_exact, pa.no_cpu_baseline, pa.model_dir = False, True, model_dir
            pf = bench_prefill(pa)
            result["prefill_4096"] = {"value": pf["value"], "unit": pf["unit"], "ms_per_prompt": pf["ms_per_step"],
                                      "roofline": pf["roofline"], "mixers": pf["mixers"],
                                      "kernels": pf["kernels"], "config": pf["config"]}
        except Exception as e:  # the decode line stands on its own
            result["prefill_4096"] = {"error": repr(e)}
    if not (small or long_ctx) and not a.no_mixer_lines:
        # the isolated mixer workloads measured in the same run: 18 GDN layers per launch
        # (state in the Infinity Cache, and 16 rotated state sets read from HBM) and 6
        # attention layers at 8k with the KV caches beyond the Infinity Cache; `--workload gdn`
        # / `--workload attn` give the full lines
        try:
            iso = {}
            for R in (1, 16):
                ga = argparse.Namespace(**vars(a))
                ga.steps, ga.warmup, ga.rotate = 64, 8, R
                g = bench_gdn(ga)
                key = "gdn_18layers_cache_resident" if R == 1 else f"gdn_18layers_{R}_state_sets"
                iso[key] = {k: {"us_per_token": v["us_per_token"], "GBs": v["GBs"], "frac": v["frac"]}
                            for k, v in g["variants"].items()}
            aa = argparse.Namespace(**vars(a))
            aa.steps, aa.warmup, aa.rotate, aa.ctx_list, aa.attn_splits = 64, 8, 8, [8192], 0
            at = bench_attn(aa)["contexts"]["8192"]
            iso["attn_6layers_8k_beyond_cache"] = {
                "kv_sets": at["kv_sets"], "kv_working_set_MiB": at["kv_working_set_MiB"],
                "one_launch_6_layers": at["batched"], "one_launch_per_layer": at["per_layer"]}
            result["isolated_mixers"] = iso
        except Exception as e:  # the decode line stands on its own
            result["isolated_mixers"] = {"error": repr(e)}
    if not (small or long_ctx) and not a.no_long_line:
        # the same decode at the end of a 131072-position arena planned by solve_max_context
        # (64 timed steps); `--workload long` gives the full line
        try:
            la = argparse.Namespace(**vars(a))
            la.workload, la.steps, la.warmup, la.no_cpu_baseline, la.model_dir = "long", 64, 8, True, ""
            la.calibration_copy = False
            lr = bench_decode(la)
            result["long_context"] = {"value": lr["value"], "unit": lr["unit"], "ms_per_step": lr["ms_per_step"],
                                      "context": lr["config"]["context"], "max_context": lr["config"]["max_context"],
                                      "roofline_attention": lr["roofline_attention"], "mixers": lr["mixers"]}
        except Exception as e:  # the decode line stands on its own
            result["long_context"] = {"error": repr(e)}
    if a.calibration_copy:
        calibration_copy()
    traffic_file = os.path.join(ROOT, "profiles", "decode_2b_8k_traffic.json")
    if os.path.exists(traffic_file) and not small and ctx == 8192 and a.kv == "fp32":
        # HBM bytes per launch from the committed FETCH_SIZE / WRITE_SIZE counter runs
        with open(traffic_file) as f:
            tr = json.load(f)
        result["roofline"]["traffic"] = tr.get("gemv_bytes_per_launch")
        result["roofline_attention"]["traffic"] = tr.get("attn_bytes_per_launch")
    if not a.no_cpu_baseline:
        with stdout_to_stderr():
            result["cpu_baseline"] = (cpu_greedy_baseline(model_dir, d, ctx, a.cpu_steps) if small
                                      else cpu_baseline(model_dir, d, ctx, a.cpu_steps))
    return result


if __name__ == "__main__":
    main()
