"""ctypes binding of libq35.so (the C ABI declared in include/q35.h) for Python callers.

The library is loaded from ``lib/libq35.so`` next to this file; importing this module
fails loudly when it has not been built. Device buffers for the kernel-level entry points
come from the HIP runtime itself (``Hip`` below), so no other GPU framework is needed.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libq35.so")
ATTN_STATIC_SCRATCH_BYTES = 8 << 20  # Q35_ATTN_STATIC_SCRATCH_BYTES of include/q35.h

Q35_OK = 0
KT_NAMES = ["gemv", "gdn_decode", "attn_decode", "attn_combine", "other", "gemm", "gdn_prefill",
            "attn_prefill"]


class Q35Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"q35 status {status}: {msg}")
        self.status = status


class Dims(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32), ("n_layers_total", C.c_int32),
        ("n_layers_gdn", C.c_int32), ("n_layers_attn", C.c_int32),
        ("gdn_k_heads", C.c_int32), ("gdn_v_heads", C.c_int32),
        ("gdn_k_head_dim", C.c_int32), ("gdn_v_head_dim", C.c_int32),
        ("gdn_conv_kernel", C.c_int32), ("attn_q_heads", C.c_int32),
        ("attn_kv_heads", C.c_int32), ("attn_head_dim", C.c_int32),
        ("ffn_intermediate", C.c_int32), ("vocab_size", C.c_int32),
        ("native_max_context", C.c_int64), ("n_params", C.c_int64),
        ("rope_theta", C.c_double), ("rms_norm_eps", C.c_float),
        ("partial_rotary_factor", C.c_float), ("attn_interval", C.c_int32),
        ("tie_word_embeddings", C.c_int32),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class Budget(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "weight_bytes", "gdn_state_bytes", "gdn_conv_bytes", "kv_cache_bytes",
        "activation_bytes", "vision_scratch_bytes", "prompt_arena_bytes")]


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.c_int64 * 4), ("data", C.c_void_p)]


class GdnDecodeArgs(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("k_heads", C.c_int32), ("v_heads", C.c_int32),
                ("head_dim_k", C.c_int32), ("head_dim_v", C.c_int32), ("conv_kernel", C.c_int32),
                ("pos", C.c_int32), ("eps", C.c_float)] + [
        (n, C.c_void_p) for n in ("qkv", "z", "b", "a", "conv_w", "A_log", "dt_bias", "norm_w",
                                  "conv_ring", "state", "out")]


class AttnDecodeArgs(C.Structure):
    _fields_ = [("q_heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("rotary_dim", C.c_int32), ("pos", C.c_int32), ("n_splits", C.c_int32),
                ("n_layers", C.c_int32), ("kv_dtype", C.c_int32), ("max_context", C.c_int64),
                ("rope_theta", C.c_double), ("eps", C.c_float)] + [
        (n, C.c_void_p) for n in ("qg", "k_new", "v_new", "q_norm", "k_norm", "k_cache",
                                  "v_cache", "out", "workspace")] + [
        ("workspace_bytes", C.c_uint64)]


class ModelOptions(C.Structure):
    _fields_ = [("kv_bytes_per_elem", C.c_int32), ("prefill_block", C.c_int32), ("prefill_exact", C.c_int32),
                ("reserved", C.c_int32 * 5)]


class GdnPrefillArgs(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_tokens", "pos0", "k_heads", "v_heads", "head_dim_k",
                                         "head_dim_v", "conv_kernel")] + [("eps", C.c_float)] + [
        (n, C.c_void_p) for n in ("qkv", "z", "b", "a")] + [
        (n, C.c_int64) for n in ("ld_qkv", "ld_z", "ld_ba")] + [
        (n, C.c_void_p) for n in ("conv_w", "A_log", "dt_bias", "norm_w", "conv_ring", "state",
                                  "out", "workspace")] + [("workspace_bytes", C.c_uint64)]


class AttnPrefillArgs(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_tokens", "pos0", "q_heads", "kv_heads", "head_dim",
                                         "rotary_dim", "kv_dtype", "reserved")] + [
        ("max_context", C.c_int64), ("rope_theta", C.c_double), ("eps", C.c_float),
        ("qkv", C.c_void_p), ("ld_qkv", C.c_int64)] + [
        (n, C.c_void_p) for n in ("q_norm", "k_norm", "k_cache", "v_cache", "out", "workspace")] + [
        ("workspace_bytes", C.c_uint64)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                          "(make -C qwen3.5-cpu-cpp_amd)")
    lib = C.CDLL(LIB_PATH)
    P, I32, I64, U64, F, D, S = (C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float,
                                 C.c_double, C.c_int32)
    sig = {
        "q35_last_error": (C.c_char_p, []),
        "q35_version": (C.c_char_p, []),
        "q35_device_alloc_count": (I64, []),
        "q35_dims_default": (None, [C.POINTER(Dims)]),
        "q35_load_config": (S, [C.c_char_p, C.POINTER(Dims)]),
        "q35_is_attention_layer": (I32, [C.POINTER(Dims), I32]),
        "q35_gdn_conv_state_bytes": (U64, [C.POINTER(Dims)]),
        "q35_compute_budget": (S, [C.POINTER(Dims), I32, I64, I32, I32, I32, C.POINTER(Budget)]),
        "q35_solve_max_context": (I64, [C.POINTER(Dims), U64, U64, U64, U64, U64, U64, I32]),
        "q35_synth_write_model": (S, [C.c_char_p, C.POINTER(Dims), U64, F, I32]),
        "q35_synth_token_ids": (S, [U64, I32, I32, P]),
        "q35_synth_normal": (S, [P, I64, U64, U64, F, I32]),
        "q35_model_create": (S, [C.POINTER(Dims), C.POINTER(Tensor), I32, I64, C.POINTER(P)]),
        "q35_model_open": (S, [C.c_char_p, I64, C.POINTER(P)]),
        "q35_model_open_opts": (S, [C.c_char_p, I64, C.POINTER(ModelOptions), C.POINTER(P)]),
        "q35_model_create_opts": (S, [C.POINTER(Dims), C.POINTER(Tensor), I32, I64, C.POINTER(ModelOptions),
                                      C.POINTER(P)]),
        "q35_model_destroy": (None, [P]),
        "q35_model_dims": (S, [P, C.POINTER(Dims)]),
        "q35_model_budget": (S, [P, C.POINTER(Budget)]),
        "q35_model_position": (I64, [P]),
        "q35_model_max_context": (I64, [P]),
        "q35_model_stream": (P, [P]),
        "q35_model_synchronize": (S, [P]),
        "q35_model_reset": (S, [P]),
        "q35_model_step": (S, [P, I32, P, P]),
        "q35_model_generate_greedy": (S, [P, P, I32, I32, P]),
        "q35_model_decode_greedy": (S, [P, I32, I32, P]),
        "q35_model_prefill": (S, [P, P, I32, P]),
        "q35_model_extend": (S, [P, P, I32, P, P]),
        "q35_model_set_prefill_block": (S, [P, I32]),
        "q35_model_set_prefill_head": (S, [P, I32]),
        "q35_model_prefill_logits_width": (I64, [P]),
        "q35_model_reserve_context": (S, [P, I64]),
        "q35_model_set_graph": (S, [P, I32]),
        "q35_model_set_layer_trace": (S, [P, I32]),
        "q35_model_read_layer_trace": (S, [P, P]),
        "q35_model_read_hidden": (S, [P, P]),
        "q35_model_set_kernel_timing": (S, [P, I32]),
        "q35_model_set_attn_splits": (S, [P, I32]),
        "q35_model_kernel_times": (S, [P, P, P]),
        "q35_model_read_gdn_state": (S, [P, I32, P]),
        "q35_model_write_gdn_state": (S, [P, I32, P]),
        "q35_model_read_conv_state": (S, [P, I32, P]),
        "q35_model_write_conv_state": (S, [P, I32, P]),
        "q35_model_read_kv": (S, [P, I32, I64, I64, P, P]),
        "q35_model_write_kv": (S, [P, I32, I64, I64, P, P]),
        "q35_model_set_position": (S, [P, I64]),
        "q35_model_fill_synthetic": (S, [P, I64, U64, F]),
        "q35_matmul_bf16": (S, [P, P, P, I32, I32, P]),
        "q35_matmul_f32": (S, [P, P, P, I32, I32, P]),
        "q35_rmsnorm": (S, [P, P, P, I32, I32, F, P]),
        "q35_rmsnorm_gated": (S, [P, P, P, P, I32, I32, F, P]),
        "q35_l2norm": (S, [P, I32, I32, F, P]),
        "q35_apply_rope": (S, [P, I32, I32, I32, P, I32, D, P]),
        "q35_gdn_decode": (S, [C.POINTER(GdnDecodeArgs), P]),
        "q35_attn_decode_workspace_bytes": (U64, [C.POINTER(AttnDecodeArgs)]),
        "q35_attn_decode": (S, [C.POINTER(AttnDecodeArgs), P]),
        "q35_attn_decode_static": (S, [C.POINTER(AttnDecodeArgs), P]),
        "q35_gemm_bf16": (S, [P, I64, P, I32, I32, I32, P, I64, P, I64, P]),
        "q35_gemm_f16x2_workspace_bytes": (U64, [I32, I32, I32]),
        "q35_gemm_f16x2": (S, [P, I64, P, I32, I32, I32, P, I64, P, I64, P, U64, P]),
        "q35_gdn_prefill_workspace_bytes": (U64, [C.POINTER(GdnPrefillArgs)]),
        "q35_gdn_prefill": (S, [C.POINTER(GdnPrefillArgs), P]),
        "q35_attn_prefill_workspace_bytes": (U64, [C.POINTER(AttnPrefillArgs)]),
        "q35_attn_prefill": (S, [C.POINTER(AttnPrefillArgs), P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(status: int) -> None:
    if status != Q35_OK:
        raise Q35Error(status, lib.q35_last_error().decode())


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ----------------------------------------------------------------------------- config
def default_dims(**over) -> Dims:
    d = Dims()
    lib.q35_dims_default(C.byref(d))
    for k, v in over.items():
        setattr(d, k, v)
    d.n_layers_attn = d.n_layers_total // d.attn_interval
    d.n_layers_gdn = d.n_layers_total - d.n_layers_attn
    return d


def load_config(path: str) -> Dims:
    d = default_dims()
    check(lib.q35_load_config(path.encode(), C.byref(d)))
    return d


def synth_write_model(directory: str, dims: Dims, seed: int = 0, std: float = 0.02,
                      threads: int = 0) -> None:
    check(lib.q35_synth_write_model(directory.encode(), C.byref(dims), seed, std, threads))


def synth_token_ids(seed: int, vocab: int, n: int) -> np.ndarray:
    ids = np.zeros(n, np.int32)
    check(lib.q35_synth_token_ids(seed, vocab, n, ptr(ids)))
    return ids


def synth_normal(n: int, seed: int, stream: int, std: float = 1.0) -> np.ndarray:
    out = np.zeros(n, np.float32)
    check(lib.q35_synth_normal(ptr(out), n, seed, stream, std, 0))
    return out


# ----------------------------------------------------------------------------- model
class Model:
    """The device-resident decoder (QwenModel on the GPU)."""

    def __init__(self, model_dir: str, max_context: int, kv_bytes_per_elem: int = 4, prefill_block: int = 0,
                 prefill_exact: bool = False):
        """max_context 0: planned by the memory equation against the device's memory;
        prefill_block > 0: the prompt arena is planned at creation for blocks of that size;
        prefill_exact: the prefill GEMMs on three exact bf16 parts (no fp16 weight copies)."""
        h = C.c_void_p()
        opt = ModelOptions(kv_bytes_per_elem=kv_bytes_per_elem, prefill_block=prefill_block,
                           prefill_exact=int(prefill_exact))
        check(lib.q35_model_open_opts(model_dir.encode(), max_context, C.byref(opt), C.byref(h)))
        self.h = h
        d = Dims()
        check(lib.q35_model_dims(h, C.byref(d)))
        self.dims = d

    def close(self):
        if self.h:
            lib.q35_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        return lib.q35_model_position(self.h)

    @property
    def max_context(self) -> int:
        return lib.q35_model_max_context(self.h)

    def budget(self) -> dict:
        b = Budget()
        check(lib.q35_model_budget(self.h, C.byref(b)))
        return {k: getattr(b, k) for k, _ in b._fields_}

    def reset(self):
        check(lib.q35_model_reset(self.h))

    def step(self, token: int, want_logits: bool = True):
        logits = np.zeros(self.dims.vocab_size, np.float32) if want_logits else None
        am = C.c_int32(0)
        check(lib.q35_model_step(self.h, int(token), ptr(logits) if want_logits else None,
                                 C.byref(am)))
        return logits, am.value

    def generate_greedy(self, prompt, n_new: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        check(lib.q35_model_generate_greedy(self.h, ptr(pr), len(pr), n_new, ptr(out)))
        return out[:n_new]

    def decode_greedy(self, token: int, n_new: int) -> np.ndarray:
        out = np.zeros(max(n_new, 1), np.int32)
        check(lib.q35_model_decode_greedy(self.h, int(token), n_new, ptr(out)))
        return out[:n_new]

    @property
    def prefill_logits_width(self) -> int:
        return lib.q35_model_prefill_logits_width(self.h)

    def set_prefill_head(self, embedding: bool):
        """Prefill logits from the embedding over all its rows (QwenForward::prefill's rule)
        instead of the step's output head."""
        check(lib.q35_model_set_prefill_head(self.h, 1 if embedding else 0))

    def reserve_context(self, max_context: int):
        check(lib.q35_model_reserve_context(self.h, int(max_context)))

    def prefill(self, ids, want_logits: bool = True):
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.zeros((len(ids), self.prefill_logits_width), np.float32) if want_logits else None
        check(lib.q35_model_prefill(self.h, ptr(ids), len(ids), ptr(lg) if want_logits else None))
        return lg

    def extend(self, ids, want_logits: bool = True, want_trace: bool = False):
        """Chunked prefill of ids at the current position; (logits [n][V], trace [n][L][H])."""
        ids = np.ascontiguousarray(ids, np.int32)
        d = self.dims
        lg = np.zeros((len(ids), self.prefill_logits_width), np.float32) if want_logits else None
        tr = np.zeros((len(ids), d.n_layers_total, d.hidden_size), np.float32) if want_trace else None
        check(lib.q35_model_extend(self.h, ptr(ids), len(ids), ptr(lg) if want_logits else None,
                                   ptr(tr) if want_trace else None))
        return lg, tr

    def set_prefill_block(self, tokens: int):
        check(lib.q35_model_set_prefill_block(self.h, int(tokens)))

    def set_graph(self, on: bool):
        check(lib.q35_model_set_graph(self.h, int(on)))

    def set_layer_trace(self, on: bool):
        check(lib.q35_model_set_layer_trace(self.h, int(on)))

    def layer_trace(self) -> np.ndarray:
        d = self.dims
        out = np.zeros((d.n_layers_total, d.hidden_size), np.float32)
        check(lib.q35_model_read_layer_trace(self.h, ptr(out)))
        return out

    def hidden(self) -> np.ndarray:
        out = np.zeros(self.dims.hidden_size, np.float32)
        check(lib.q35_model_read_hidden(self.h, ptr(out)))
        return out

    def set_kernel_timing(self, on: bool):
        check(lib.q35_model_set_kernel_timing(self.h, int(on)))

    def set_attn_splits(self, n: int):
        check(lib.q35_model_set_attn_splits(self.h, n))

    def kernel_times(self) -> dict:
        ms = np.zeros(len(KT_NAMES), np.float64)
        n = np.zeros(len(KT_NAMES), np.int64)
        check(lib.q35_model_kernel_times(self.h, ptr(ms), ptr(n)))
        return {k: (float(ms[i]), int(n[i])) for i, k in enumerate(KT_NAMES)}

    def _conv_dim(self):
        d = self.dims
        return 2 * d.gdn_k_heads * d.gdn_k_head_dim + d.gdn_v_heads * d.gdn_v_head_dim

    def gdn_state(self, layer: int) -> np.ndarray:
        d = self.dims
        out = np.zeros((d.gdn_v_heads, d.gdn_k_head_dim, d.gdn_v_head_dim), np.float32)
        check(lib.q35_model_read_gdn_state(self.h, layer, ptr(out)))
        return out

    def set_gdn_state(self, layer: int, s: np.ndarray):
        s = np.ascontiguousarray(s, np.float32)
        check(lib.q35_model_write_gdn_state(self.h, layer, ptr(s)))

    def conv_state(self, layer: int) -> np.ndarray:
        out = np.zeros((self._conv_dim(), self.dims.gdn_conv_kernel - 1), np.float32)
        check(lib.q35_model_read_conv_state(self.h, layer, ptr(out)))
        return out

    def set_conv_state(self, layer: int, w: np.ndarray):
        w = np.ascontiguousarray(w, np.float32)
        check(lib.q35_model_write_conv_state(self.h, layer, ptr(w)))

    def kv(self, layer: int, pos0: int, n: int):
        d = self.dims
        k = np.zeros((n, d.attn_kv_heads, d.attn_head_dim), np.float32)
        v = np.zeros_like(k)
        check(lib.q35_model_read_kv(self.h, layer, pos0, n, ptr(k), ptr(v)))
        return k, v

    def set_kv(self, layer: int, pos0: int, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        check(lib.q35_model_write_kv(self.h, layer, pos0, k.shape[0], ptr(k), ptr(v)))

    def set_position(self, pos: int):
        check(lib.q35_model_set_position(self.h, pos))

    def fill_synthetic(self, pos: int, seed: int = 0, state_std: float = 0.1):
        check(lib.q35_model_fill_synthetic(self.h, pos, seed, state_std))


# ----------------------------------------------------------------------------- HIP runtime
class Hip:
    """Minimal HIP runtime access (device buffers, streams, events) through ctypes."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
        r = self.rt
        P = C.c_void_p
        for name, args in {
            "hipMalloc": [C.POINTER(P), C.c_size_t],
            "hipFree": [P],
            "hipMemcpy": [P, P, C.c_size_t, C.c_int],
            "hipMemset": [P, C.c_int, C.c_size_t],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [P],
            "hipStreamCreate": [C.POINTER(P)],
            "hipStreamDestroy": [P],
            "hipEventCreate": [C.POINTER(P)],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [C.POINTER(C.c_float), P, P],
            "hipGetDeviceCount": [C.POINTER(C.c_int)],
            "hipMemGetInfo": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)],
            "hipGetErrorString": [C.c_int],
        }.items():
            fn = getattr(r, name)
            fn.argtypes = args
            fn.restype = C.c_char_p if name == "hipGetErrorString" else C.c_int

    def _ck(self, e, what):
        if e != 0:
            raise RuntimeError(f"{what} failed: {self.rt.hipGetErrorString(e).decode()}")

    def device_count(self) -> int:
        n = C.c_int(0)
        e = self.rt.hipGetDeviceCount(C.byref(n))
        return n.value if e == 0 else 0

    def mem_info(self):
        """(free, total) bytes of the current device."""
        f, t = C.c_size_t(0), C.c_size_t(0)
        self._ck(self.rt.hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
        return f.value, t.value

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self._ck(self.rt.hipMalloc(C.byref(p), max(int(nbytes), 1)), "hipMalloc")
        return p.value

    def free(self, p: int):
        self._ck(self.rt.hipFree(C.c_void_p(p)), "hipFree")

    def upload(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        p = self.malloc(a.nbytes)
        self._ck(self.rt.hipMemcpy(C.c_void_p(p), C.c_void_p(a.ctypes.data), a.nbytes, 1), "hipMemcpy H2D")
        return p

    def copy_in(self, p: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self._ck(self.rt.hipMemcpy(C.c_void_p(p), C.c_void_p(a.ctypes.data), a.nbytes, 1), "hipMemcpy H2D")

    def download(self, p: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._ck(self.rt.hipMemcpy(C.c_void_p(out.ctypes.data), C.c_void_p(p), out.nbytes, 2), "hipMemcpy D2H")
        return out

    def sync(self):
        self._ck(self.rt.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream_sync(self, s):
        self._ck(self.rt.hipStreamSynchronize(C.c_void_p(s)), "hipStreamSynchronize")

    def event(self) -> int:
        e = C.c_void_p()
        self._ck(self.rt.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream=None):
        self._ck(self.rt.hipEventRecord(C.c_void_p(ev), C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b) -> float:
        self._ck(self.rt.hipEventSynchronize(C.c_void_p(b)), "hipEventSynchronize")
        ms = C.c_float(0)
        self._ck(self.rt.hipEventElapsedTime(C.byref(ms), C.c_void_p(a), C.c_void_p(b)), "hipEventElapsedTime")
        return ms.value


def dims_for(name: str) -> Dims:
    """Named shapes used by the tests and the benchmark."""
    if name == "tiny":
        return default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                            attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=512,
                            vocab_size=1024, native_max_context=4096)
    if name == "tiny_untied":  # separate lm_head: greedy ids follow the context
        return default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=2, gdn_v_heads=2,
                            attn_q_heads=2, attn_kv_heads=1, ffn_intermediate=512,
                            vocab_size=1024, native_max_context=4096, tie_word_embeddings=0)
    if name == "tiny_gqa":  # v-heads = 2 x k-heads, GQA group 4
        return default_dims(hidden_size=256, n_layers_total=4, gdn_k_heads=1, gdn_v_heads=2,
                            attn_q_heads=4, attn_kv_heads=1, ffn_intermediate=512,
                            vocab_size=1024, native_max_context=4096)
    if name == "0.8b":
        return default_dims(hidden_size=1024, n_layers_total=24, ffn_intermediate=3584,
                            vocab_size=151936, native_max_context=262144)
    if name == "2b":
        return default_dims(hidden_size=2048, n_layers_total=24, attn_q_heads=16,
                            attn_kv_heads=2, ffn_intermediate=6144, vocab_size=151936,
                            native_max_context=262144)
    raise KeyError(name)
