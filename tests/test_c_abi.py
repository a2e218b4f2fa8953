"""libq35.so on the host: it loads, exports every entry point include/q35.h declares, and its
host-only parts (config reader, memory equation, synthetic writer, argument checks and
error reporting) behave like the reference's. No GPU work is started here."""
import ctypes as C
import json
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import golden, read_safetensors, sha256

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q35.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q35_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) > 40
    out = subprocess.run(["nm", "-D", "--defined-only", pyq35.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (q35_\w+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    for s in syms:  # and ctypes resolves each of them from the loaded library
        getattr(pyq35.lib, s)


def test_version_and_error_channel():
    assert b"gfx950" in pyq35.lib.q35_version()
    st = pyq35.lib.q35_load_config(b"/nonexistent/config.json", C.byref(pyq35.default_dims()))
    assert st == -3
    assert b"cannot open" in pyq35.lib.q35_last_error()


def test_default_dims_match_reference_defaults():
    d = pyq35.default_dims()
    assert (d.hidden_size, d.n_layers_total, d.n_layers_gdn, d.n_layers_attn) == (1024, 24, 18, 6)
    assert (d.gdn_k_heads, d.gdn_v_heads, d.gdn_k_head_dim, d.gdn_v_head_dim, d.gdn_conv_kernel) == (16, 16, 128, 128, 4)
    assert (d.attn_q_heads, d.attn_kv_heads, d.attn_head_dim) == (8, 2, 256)
    assert (d.ffn_intermediate, d.vocab_size, d.native_max_context) == (3584, 248320, 262144)
    assert d.rope_theta == 1e7 and d.attn_interval == 4 and d.tie_word_embeddings == 1
    assert abs(d.partial_rotary_factor - 0.25) < 1e-9 and abs(d.rms_norm_eps - 1e-6) < 1e-12
    for layer in range(24):
        assert pyq35.lib.q35_is_attention_layer(C.byref(d), layer) == int((layer + 1) % 4 == 0)


def test_config_reader(tmp_path):
    cfg = tmp_path / "config.json"
    cfg.write_text('{"vision_config": {"hidden_size": 1152}, "text_config": {"hidden_size": 2048,'
                   ' "num_hidden_layers": 8, "linear_num_value_heads": 32, "head_dim": 256,'
                   ' "linear_key_head_dim": 128, "rope_parameters": {"rope_theta": 5000000,'
                   ' "partial_rotary_factor": 0.5}, "rms_norm_eps": 1e-05, "vocab_size": 1000,'
                   ' "tie_word_embeddings": false, "intermediate_size": 6144}}')
    d = pyq35.load_config(str(cfg))
    assert (d.hidden_size, d.n_layers_total, d.n_layers_attn, d.n_layers_gdn) == (2048, 8, 2, 6)
    assert (d.gdn_v_heads, d.vocab_size, d.ffn_intermediate, d.tie_word_embeddings) == (32, 1000, 6144, 0)
    assert d.rope_theta == 5e6 and abs(d.partial_rotary_factor - 0.5) < 1e-9
    assert abs(d.rms_norm_eps - 1e-5) < 1e-12
    assert d.n_params == 1000 * 2048 + 8 * 12 * 2048 * 2048
    o = op.OrcDims()
    op.olib.orc_dims_default(C.byref(o))
    assert op.olib.orc_load_config(str(cfg).encode(), C.byref(o)) == 0
    for k, _ in op.OrcDims._fields_:
        assert getattr(o, k) == pytest.approx(getattr(d, k)), k
    if op.ref_available():
        v = np.zeros(16, np.int64)
        th, eps, pf = C.c_double(), C.c_float(), C.c_float()
        op.Ref.lib().ref_config(str(cfg).encode(), v.ctypes.data, C.byref(th), C.byref(eps), C.byref(pf))
        mine = [d.hidden_size, d.n_layers_total, d.n_layers_gdn, d.n_layers_attn, d.gdn_k_heads,
                d.gdn_v_heads, d.gdn_k_head_dim, d.gdn_v_head_dim, d.gdn_conv_kernel, d.attn_q_heads,
                d.attn_kv_heads, d.attn_head_dim, d.ffn_intermediate, d.vocab_size,
                d.native_max_context, d.n_params]
        assert v.tolist() == mine
        assert th.value == d.rope_theta and eps.value == d.rms_norm_eps


QUIRKY_CONFIGS = [
    # flat file (no text_config), integers rounded as (int)(v + 0.5), exponents
    '{"hidden_size": 2047.6, "num_hidden_layers": 8.4, "vocab_size": 1e3, "rms_norm_eps": 1E-5}',
    # "true" after the flag's comma does not count; the first occurrence of a key wins,
    # nested objects included; a key quoted as a string value is still the key's first match
    '{"text_config": {"tie_word_embeddings": false, "x": true, "rope_parameters": {"rope_theta": 25e4},'
    ' "rope_theta": 1, "model_type": "head_dim", "head_dim": 128}}',
    # out-of-range and malformed numbers keep the defaults; blanks before the value
    '{"text_config": {"hidden_size": 1e999, "intermediate_size": -, "vocab_size":\n\t 512,'
    ' "partial_rotary_factor": 5e-400, "tie_word_embeddings": true}}',
    # an unterminated text_config object: the whole file is the scope
    '{"hidden_size": 64, "text_config": {"hidden_size": 32',
]


@pytest.mark.skipif(not op.ref_available(), reason="reference build absent")
@pytest.mark.parametrize("text", QUIRKY_CONFIGS)
def test_config_reader_quirks_match_reference(tmp_path, text):
    """The reader's textual lookup rules on unusual files, side by side with the compiled
    reference loader (src/config_loader.cpp:13-108)."""
    cfg = tmp_path / "config.json"
    cfg.write_text(text)
    d = pyq35.load_config(str(cfg))
    v = np.zeros(16, np.int64)
    th, eps, pf = C.c_double(), C.c_float(), C.c_float()
    op.Ref.lib().ref_config(str(cfg).encode(), v.ctypes.data, C.byref(th), C.byref(eps), C.byref(pf))
    mine = [d.hidden_size, d.n_layers_total, d.n_layers_gdn, d.n_layers_attn, d.gdn_k_heads,
            d.gdn_v_heads, d.gdn_k_head_dim, d.gdn_v_head_dim, d.gdn_conv_kernel, d.attn_q_heads,
            d.attn_kv_heads, d.attn_head_dim, d.ffn_intermediate, d.vocab_size,
            d.native_max_context, d.n_params]
    assert v.tolist() == mine
    assert th.value == d.rope_theta and eps.value == pytest.approx(d.rms_norm_eps, rel=1e-7)
    assert pf.value == pytest.approx(d.partial_rotary_factor, rel=1e-7)


def _budget(d, bpw, ctx, kvb):
    b = pyq35.Budget()
    pyq35.check(pyq35.lib.q35_compute_budget(C.byref(d), bpw, ctx, kvb, 4, 1024, C.byref(b)))
    return b


def test_memory_equation_closed_form():
    d = pyq35.dims_for("2b")
    b = _budget(d, 2, 131072, 4)
    assert b.kv_cache_bytes == 6 * 131072 * 2 * 2 * 256 * 4 == 3221225472
    assert b.gdn_state_bytes == 18 * 16 * 128 * 128 * 4 == 18874368
    assert b.gdn_conv_bytes == 18 * 6144 * 3 * 4 == 1327104
    assert pyq35.lib.q35_gdn_conv_state_bytes(C.byref(d)) == 1327104
    assert b.weight_bytes == d.n_params * 2
    assert b.activation_bytes == max(6144 * 4 * 2, (16 * 256 + 2 * 2 * 256) * 4, 3 * 16 * 128 * 4)
    assert b.vision_scratch_bytes == 4 * 256 * 1024 * 4 + 256 * 1024 * 4 * 2
    # reverse solve: 288 GB leaves room for ~11.7M positions, clamped to the native cap
    ram = 288 * 10**9
    ctx = pyq35.lib.q35_solve_max_context(C.byref(d), ram, b.weight_bytes, b.gdn_state_bytes,
                                          b.activation_bytes, 0, 1 << 30, 4)
    assert ctx == d.native_max_context
    d131 = pyq35.dims_for("2b")
    d131.native_max_context = 131072
    assert pyq35.lib.q35_solve_max_context(C.byref(d131), ram, b.weight_bytes, b.gdn_state_bytes,
                                           b.activation_bytes, 0, 1 << 30, 4) == 131072
    d.native_max_context = 2**31 - 1  # ModelConfig keeps the cap in an int
    per_tok = 6 * 2 * 2 * 256 * 4
    fixed = b.weight_bytes + b.gdn_state_bytes + b.activation_bytes + (1 << 30)
    assert pyq35.lib.q35_solve_max_context(C.byref(d), ram, b.weight_bytes, b.gdn_state_bytes,
                                           b.activation_bytes, 0, 1 << 30, 4) == (ram - fixed) // per_tok
    assert pyq35.lib.q35_solve_max_context(C.byref(d), 1000, 2000, 0, 0, 0, 0, 4) == -1


@pytest.mark.skipif(not op.ref_available(), reason="reference build absent")
def test_memory_equation_matches_reference(tmp_path):
    d = pyq35.dims_for("2b")
    pyq35.synth_write_model(str(tmp_path), pyq35.dims_for("tiny"), 0)
    cfgp = str(tmp_path / "config.json")
    dt = pyq35.load_config(cfgp)
    for ctx, kvb, bpw in [(1, 4, 2), (4096, 2, 1), (131072, 4, 2)]:
        mine = _budget(dt, bpw, ctx, kvb)
        out = np.zeros(6, np.uint64)
        op.Ref.lib().ref_budget(cfgp.encode(), bpw, ctx, kvb, out.ctypes.data)
        assert [getattr(mine, k) for k, _ in mine._fields_[:6]] == out.tolist()
        assert mine.prompt_arena_bytes == 0  # the reference has no prompt arena
    args = (10**11, 5 * 10**9, 10**8, 10**7, 0, 10**9, 4)
    assert pyq35.lib.q35_solve_max_context(C.byref(dt), *args) == \
        op.Ref.lib().ref_solve_max_context(cfgp.encode(), *args)
    del d


def test_synthetic_writer_deterministic(tmp_path):
    d = pyq35.dims_for("tiny")
    pyq35.synth_write_model(str(tmp_path / "a"), d, seed=0, threads=1)
    pyq35.synth_write_model(str(tmp_path / "b"), d, seed=0, threads=7)
    ha = sha256(str(tmp_path / "a" / "model.safetensors"))
    assert ha == sha256(str(tmp_path / "b" / "model.safetensors")) == str(golden("tiny")["sha256"])
    pyq35.synth_write_model(str(tmp_path / "c"), d, seed=1)
    assert sha256(str(tmp_path / "c" / "model.safetensors")) != ha
    # the values are N(0, 0.02) draws; (1+w) norms are 0 and the GDN gated-norm weight 1
    t = read_safetensors(str(tmp_path / "a" / "model.safetensors"))
    emb = (t["model.language_model.embed_tokens.weight"].astype(np.uint32) << 16).view(np.float32)
    assert abs(emb.std() - 0.02) < 0.001 and abs(emb.mean()) < 0.001
    gn = t["model.language_model.layers.0.linear_attn.norm.weight"]
    assert (gn == 0x3F80).all()
    assert (t["model.language_model.layers.0.input_layernorm.weight"] == 0).all()
    ids = pyq35.synth_token_ids(1, 1000, 64)
    assert ids.min() >= 0 and ids.max() < 1000
    np.testing.assert_array_equal(ids, pyq35.synth_token_ids(1, 1000, 64))


def _table(model_dir, drop=None):
    ts = read_safetensors(os.path.join(model_dir, "model.safetensors"))
    keep, arrs = [], []
    for name, arr in ts.items():
        if name == drop:
            continue
        arr = np.ascontiguousarray(arr)
        t = pyq35.Tensor()
        t.name = name.encode()
        t.dtype = 0 if arr.dtype == np.uint16 else 1
        t.ndim = arr.ndim
        for i, s in enumerate(arr.shape):
            t.shape[i] = s
        t.data = arr.ctypes.data
        keep.append(t)
        arrs.append(arr)
    return (pyq35.Tensor * len(keep))(*keep), arrs


def test_model_create_reports_missing_weight(model_dirs):
    """The weight plan is checked before any device work: a missing tensor fails cleanly."""
    d = pyq35.dims_for("tiny")
    name = "model.language_model.layers.1.linear_attn.A_log"
    tab, keep = _table(model_dirs["tiny"], drop=name)
    h = C.c_void_p()
    st = pyq35.lib.q35_model_create(C.byref(d), tab, len(tab), 64, C.byref(h))
    assert st == -5 and not h.value
    assert name.encode() in pyq35.lib.q35_last_error()


def test_model_create_rejects_unsupported_shapes(model_dirs):
    d = pyq35.dims_for("tiny")
    d.gdn_k_head_dim = 64
    tab, keep = _table(model_dirs["tiny"])
    h = C.c_void_p()
    assert pyq35.lib.q35_model_create(C.byref(d), tab, len(tab), 64, C.byref(h)) == -7
    d = pyq35.dims_for("tiny")
    d.attn_q_heads = 3
    assert pyq35.lib.q35_model_create(C.byref(d), tab, len(tab), 64, C.byref(h)) == -7
    d = pyq35.dims_for("tiny")
    assert pyq35.lib.q35_model_create(C.byref(d), tab, len(tab), -1, C.byref(h)) == -6
    opt = pyq35.ModelOptions(kv_bytes_per_elem=1)
    assert pyq35.lib.q35_model_create_opts(C.byref(d), tab, len(tab), 64, C.byref(opt), C.byref(h)) == -7
    assert b"KV cache element" in pyq35.lib.q35_last_error()


def test_model_open_reports_bad_files(tmp_path, model_dirs):
    h = C.c_void_p()
    assert pyq35.lib.q35_model_open(str(tmp_path / "none").encode(), 64, C.byref(h)) == -3
    # truncated shard
    bad = tmp_path / "trunc"
    shutil.copytree(model_dirs["tiny"], bad)
    p = bad / "model.safetensors"
    data = p.read_bytes()
    p.write_bytes(data[: len(data) // 2])
    assert pyq35.lib.q35_model_open(str(bad).encode(), 64, C.byref(h)) == -3
    # header length beyond the file
    p.write_bytes((10**12).to_bytes(8, "little") + data[8:64])
    assert pyq35.lib.q35_model_open(str(bad).encode(), 64, C.byref(h)) == -3
    # a shape whose element count wraps around 64 bits to the span's size:
    # (2^62 + 1) x 4 = 2^64 + 4 -> 4 elements of 2 bytes = the 8-byte span
    hdr = json.dumps({"w": {"dtype": "BF16", "shape": [2**62 + 1, 4], "data_offsets": [0, 8]}}).encode()
    p.write_bytes(len(hdr).to_bytes(8, "little") + hdr + bytes(8))
    assert pyq35.lib.q35_model_open(str(bad).encode(), 64, C.byref(h)) == -3
    assert not h.value


def test_kernel_entry_points_validate_before_launch():
    a = pyq35.GdnDecodeArgs(n_layers=1, k_heads=16, v_heads=16, head_dim_k=64, head_dim_v=128,
                            conv_kernel=4)
    assert pyq35.lib.q35_gdn_decode(C.byref(a), None) == -7
    at = pyq35.AttnDecodeArgs(q_heads=8, kv_heads=2, head_dim=128)
    assert pyq35.lib.q35_attn_decode(C.byref(at), None) == -7
    at = pyq35.AttnDecodeArgs(q_heads=8, kv_heads=2, head_dim=256, rotary_dim=64, pos=5,
                              max_context=4)
    assert pyq35.lib.q35_attn_decode(C.byref(at), None) == -6
    # cache element type: only 0 (fp32) and 1 (bf16); pointers are never dereferenced
    fake = dict(qg=1 << 20, k_new=1 << 20, v_new=1 << 20, q_norm=1 << 20, k_norm=1 << 20,
                k_cache=1 << 20, v_cache=1 << 20, out=1 << 20, workspace=1 << 20)
    at = pyq35.AttnDecodeArgs(q_heads=8, kv_heads=2, head_dim=256, rotary_dim=64, pos=1, max_context=4,
                              kv_dtype=2, workspace_bytes=1 << 30, **fake)
    assert pyq35.lib.q35_attn_decode(C.byref(at), None) == -1
    assert b"kv_dtype" in pyq35.lib.q35_last_error()
    ap = pyq35.AttnPrefillArgs(n_tokens=1, q_heads=8, kv_heads=2, head_dim=256, rotary_dim=64, kv_dtype=-1,
                               max_context=4, ld_qkv=5120, workspace_bytes=1 << 30,
                               **{k: v for k, v in fake.items() if k not in ("qg", "k_new", "v_new")},
                               qkv=1 << 20)
    assert pyq35.lib.q35_attn_prefill(C.byref(ap), None) == -1
    assert b"kv_dtype" in pyq35.lib.q35_last_error()
    # workspace: the full size holds the pre-split K / V tiles of an fp32 cache (3 KB per
    # position and kv head, 32-position tiles); below the Q parts alone, or misaligned: refused
    ap.kv_dtype, ap.n_tokens, ap.pos0, ap.max_context = 0, 40, 30, 128
    q_only = 8 * 40 * 256 * 4 + 256
    assert pyq35.lib.q35_attn_prefill_workspace_bytes(C.byref(ap)) == q_only + 2 * 3 * 96 * 1024
    ap.kv_dtype = 1
    assert pyq35.lib.q35_attn_prefill_workspace_bytes(C.byref(ap)) == q_only
    ap.workspace_bytes = q_only - 4
    assert pyq35.lib.q35_attn_prefill(C.byref(ap), None) == -1
    assert b"workspace of" in pyq35.lib.q35_last_error()
    ap.workspace_bytes, ap.workspace = q_only, (1 << 20) + 8
    assert pyq35.lib.q35_attn_prefill(C.byref(ap), None) == -1
    assert b"aligned" in pyq35.lib.q35_last_error()
    assert pyq35.lib.q35_matmul_bf16(None, None, None, 4, 8, None) == -1
    assert pyq35.lib.q35_matmul_bf16(1 << 20, 1 << 20, 1 << 20, 4, 12, None) == -7
    # GDN prefill: the conv pass reads qkv rows, the ring and the taps 16 bytes at a time
    gfake = {k: 1 << 20 for k in ("qkv", "z", "b", "a", "conv_w", "A_log", "dt_bias", "norm_w",
                                  "conv_ring", "state", "out", "workspace")}
    gp = pyq35.GdnPrefillArgs(n_tokens=8, k_heads=2, v_heads=2, head_dim_k=128, head_dim_v=128, conv_kernel=4,
                              ld_qkv=768, ld_z=256, ld_ba=2, **gfake)
    gp.workspace_bytes = pyq35.lib.q35_gdn_prefill_workspace_bytes(C.byref(gp))
    assert gp.workspace_bytes > 0
    for field, bad_value in (("ld_qkv", 770), ("qkv", (1 << 20) + 4), ("conv_ring", (1 << 20) + 8),
                             ("conv_w", (1 << 20) + 12), ("workspace", (1 << 20) + 4)):
        good = getattr(gp, field)
        setattr(gp, field, bad_value)
        assert pyq35.lib.q35_gdn_prefill(C.byref(gp), None) == -1, field
        assert b"16-byte aligned" in pyq35.lib.q35_last_error()
        setattr(gp, field, good)
    gp.workspace_bytes -= 4
    assert pyq35.lib.q35_gdn_prefill(C.byref(gp), None) == -1
    assert b"workspace of" in pyq35.lib.q35_last_error()


def test_attn_decode_static_refuses_oversized_partials():
    """The no-allocation attention decode checks its split-K partials against the static
    device array before any device call: beyond Q35_ATTN_STATIC_SCRATCH_BYTES it fails with
    Q35_ERR_RANGE (the pointers below are never dereferenced)."""
    fake = dict(qg=1 << 20, k_new=1 << 20, v_new=1 << 20, q_norm=1 << 20, k_norm=1 << 20,
                k_cache=1 << 20, v_cache=1 << 20, out=1 << 20)
    at = pyq35.AttnDecodeArgs(q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64, pos=10, n_splits=4096,
                              n_layers=2, max_context=1 << 20, **fake)
    hdr = open(os.path.join(ROOT, "include", "q35.h")).read()
    m = re.search(r"#define Q35_ATTN_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)", hdr)
    assert m and int(m.group(1)) << int(m.group(2)) == pyq35.ATTN_STATIC_SCRATCH_BYTES
    assert pyq35.lib.q35_attn_decode_workspace_bytes(C.byref(at)) > pyq35.ATTN_STATIC_SCRATCH_BYTES
    assert pyq35.lib.q35_attn_decode_static(C.byref(at), None) == -6
    assert b"static scratch" in pyq35.lib.q35_last_error()
    at.head_dim = 128  # shape checks as q35_attn_decode's
    assert pyq35.lib.q35_attn_decode_static(C.byref(at), None) == -7


CALLER = os.path.join(ROOT, "tests", "cpp", "forward_pass_caller")


def test_forward_pass_dropin_links_and_exports():
    """A caller written against the reference's forward_pass.h (include/forward_pass.h:21-54)
    compiles with the host compiler and links against libq35.so, which exports the six
    functions with the reference's C++ signatures; its inline activations equal the oracle's."""
    assert os.path.exists(CALLER), "tests/cpp/forward_pass_caller is not built (make -C tests/cpp)"
    out = subprocess.run(["nm", "-DC", "--defined-only", pyq35.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    for sig in ("l2norm(float*, int, float)", "matmul(float const*, float const*, float*, int, int)",
                "matmul(WeightView const&, float const*, float*, int, int)",
                "rmsnorm(float const*, float const*, float*, int, float)",
                "rmsnorm_gated(float const*, float const*, float const*, float*, int, float)",
                "apply_rope(float*, int, int, double)"):
        assert sig in out, sig
    r = subprocess.run([CALLER, "--host-only"], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
