"""The library's host-side readers and planner built with AddressSanitizer and UBSan (g++,
the host sources only; tests/cpp/host_sanitize.cpp): config.json files the reader must
handle (quirky, malformed, truncated), safetensors files with every accessor exercised on
every tensor, crafted bad headers that must be refused, and the memory equation over a range
of contexts. Any sanitizer report fails the run. CPU only."""
import json
import os
import shutil
import subprocess

import pytest

import pyq35
from test_c_abi import QUIRKY_CONFIGS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
EXE = os.path.join(CPP, "host_sanitize")


@pytest.fixture(scope="module")
def exe():
    subprocess.run(["make", "-C", CPP, "host_sanitize"], check=True, capture_output=True)
    return EXE


def run(exe, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
    p = subprocess.run([exe] + args, capture_output=True, text=True, env=env, timeout=300)
    assert "Sanitizer" not in p.stderr and "runtime error" not in p.stderr, p.stderr[-4000:]
    assert p.returncode == 0, (p.returncode, p.stderr[-4000:])
    return p.stdout.splitlines()


def write_header(path, header, data=b"", length=None):
    hdr = json.dumps(header).encode() if isinstance(header, dict) else header
    n = len(hdr) if length is None else length
    path.write_bytes(n.to_bytes(8, "little") + hdr + data)


def test_config_reader_under_sanitizers(exe, tmp_path):
    texts = QUIRKY_CONFIGS + [
        "", "{", "}", '"', '{"text_config":', '{"hidden_size": }', '{"hidden_size": 1' + "0" * 400 + "}",
        '{"text_config": {"text_config": {"hidden_size": 12}}}', "\x00\x01\x02binary" * 50,
        '{"vocab_size": 99999999999999999999, "num_hidden_layers": -4, "head_dim": 0}',
        "[" * 2000 + "]" * 2000, '{"tie_word_embeddings":' + " " * 5000,
    ]
    args = []
    for i, t in enumerate(texts):
        p = tmp_path / f"c{i}.json"
        p.write_bytes(t.encode("latin-1"))
        args.append(f"cfg:{p}")
    args.append(f"cfg:{tmp_path / 'missing.json'}")
    out = run(exe, args)
    assert len(out) == len(args)
    assert out[-1].startswith("cfg 0 ")  # a missing file is reported, the defaults kept
    assert all(o.startswith("cfg 1 ") for o in out[:-1])


def test_safetensors_reader_under_sanitizers(exe, tmp_path):
    good = tmp_path / "tiny"
    pyq35.synth_write_model(str(good), pyq35.dims_for("tiny"), seed=0, std=0.02)
    shard = good / "model.safetensors"
    data = shard.read_bytes()
    bad = []

    def case(name, blob):
        d = tmp_path / name
        d.mkdir()
        (d / "model.safetensors").write_bytes(blob)
        bad.append(f"st:{d}")

    case("trunc", data[: len(data) // 2])
    case("short", data[:5])
    case("empty", b"")
    case("hdr_beyond", (10**12).to_bytes(8, "little") + data[8:64])
    case("hdr_zero", (0).to_bytes(8, "little") + data[8:])
    for name, header, payload in [
        ("badjson", b'{"w": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]', bytes(8)),
        ("wrap", {"w": {"dtype": "BF16", "shape": [2**62 + 1, 4], "data_offsets": [0, 8]}}, bytes(8)),
        ("negshape", {"w": {"dtype": "F32", "shape": [-1, 4], "data_offsets": [0, 16]}}, bytes(16)),
        ("reversed", {"w": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}}, bytes(8)),
        ("past_end", {"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, bytes(8)),
        ("size_mismatch", {"w": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, bytes(16)),
        ("huge_dim", {"w": {"dtype": "BF16", "shape": [2**40, 2**40], "data_offsets": [0, 8]}}, bytes(8)),
    ]:
        blob_dir = tmp_path / name
        blob_dir.mkdir()
        write_header(blob_dir / "model.safetensors", header, payload)
        bad.append(f"st:{blob_dir}")
    # accepted as the reference's reader accepts them, and read without touching memory
    # they do not own: a tensor of an unknown dtype (listed, not widened) and one without a
    # shape (no elements, as the reference's numel() counts it)
    odd = tmp_path / "odd"
    odd.mkdir()
    write_header(odd / "model.safetensors",
                 {"q": {"dtype": "Q7", "shape": [2], "data_offsets": [0, 2]},
                  "s": {"dtype": "F32", "data_offsets": [2, 6]}}, bytes(6))
    # a second, valid shard next to the first: both are read
    two = tmp_path / "two"
    shutil.copytree(good, two)
    write_header(two / "z-extra.safetensors",
                 {"extra.weight": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}},
                 bytes(24))
    out = run(exe, [f"st:{good}", f"st:{shard}", f"st:{two}"] + bad + [f"st:{tmp_path / 'none'}", f"st:{odd}"])
    assert out[-1].startswith("st 1 tensors=2 ")
    out = out[:-1]
    assert out[0].startswith("st 1 ") and out[1].startswith("st 1 ")
    n_good = int(out[0].split("tensors=")[1].split()[0])
    assert n_good > 40 and f"table={n_good}" in out[0]
    assert out[2].startswith("st 1 ") and f"tensors={n_good + 1}" in out[2]
    assert not any("accepted" in o or "mismatch" in o for o in out)
    refused = [o for o in out[3:] if o.startswith("st ")]
    assert len(refused) == len(bad) + 1 and all(o.startswith("st 0 ") for o in refused), refused


def config_text(d):
    return json.dumps({"text_config": {
        "hidden_size": d.hidden_size, "num_hidden_layers": d.n_layers_total,
        "full_attention_interval": d.attn_interval, "num_attention_heads": d.attn_q_heads,
        "num_key_value_heads": d.attn_kv_heads, "head_dim": d.attn_head_dim,
        "linear_num_key_heads": d.gdn_k_heads, "linear_num_value_heads": d.gdn_v_heads,
        "linear_key_head_dim": d.gdn_k_head_dim, "linear_value_head_dim": d.gdn_v_head_dim,
        "linear_conv_kernel_dim": d.gdn_conv_kernel, "intermediate_size": d.ffn_intermediate,
        "vocab_size": d.vocab_size, "max_position_embeddings": d.native_max_context,
        "rms_norm_eps": d.rms_norm_eps, "rope_parameters": {"rope_theta": d.rope_theta,
        "partial_rotary_factor": d.partial_rotary_factor},
        "tie_word_embeddings": bool(d.tie_word_embeddings)}})


def test_memory_equation_under_sanitizers(exe, tmp_path):
    args = []
    for name in ("tiny", "0.8b", "2b"):
        p = tmp_path / f"{name}.json"
        p.write_text(config_text(pyq35.dims_for(name)))
        args.append(f"budget:{p}")
    out = run(exe, args)
    assert len(out) == 3 * 8
    for line in out:
        fields = dict(kv.split("=") for kv in line.split()[1:])
        assert int(fields["max_ctx"]) > 0 and int(fields["total"]) >= int(fields["kv"])
