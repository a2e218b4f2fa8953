"""ctypes bindings of the CPU checkers (test infrastructure only).

``Oracle`` wraps liboracle.so, the repository's CPU fp32 restatement of the reference path.
``Ref`` wraps _ref/libq35ref.so, the unmodified reference engine compiled from its own
sources by this directory's Makefile (present only where that build ran).
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libq35ref.so")


def _p(a):
    return None if a is None else a.ctypes.data


class OrcDims(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden_size", "n_layers_total", "n_layers_gdn", "n_layers_attn", "gdn_k_heads",
        "gdn_v_heads", "gdn_k_head_dim", "gdn_v_head_dim", "gdn_conv_kernel", "attn_q_heads",
        "attn_kv_heads", "attn_head_dim", "ffn_intermediate", "vocab_size")] + [
        ("native_max_context", C.c_int64), ("n_params", C.c_int64), ("rope_theta", C.c_double),
        ("rms_norm_eps", C.c_float), ("partial_rotary_factor", C.c_float),
        ("attn_interval", C.c_int32), ("tie_word_embeddings", C.c_int32)]


def _load_oracle():
    if not os.path.exists(ORACLE_PATH):
        raise ImportError(f"{ORACLE_PATH} missing: run make -C oracle")
    lib = C.CDLL(ORACLE_PATH)
    P, I, F, D = C.c_void_p, C.c_int, C.c_float, C.c_double
    sig = {
        "orc_matmul_bf16": (None, [P, P, P, I, I]),
        "orc_rmsnorm": (None, [P, P, P, I, F]),
        "orc_rmsnorm_gated": (None, [P, P, P, P, I, F]),
        "orc_l2norm": (None, [P, I, F]),
        "orc_apply_rope": (None, [P, I, I, D]),
        "orc_silu": (F, [F]), "orc_sigmoid": (F, [F]), "orc_softplus": (F, [F]),
        "orc_dims_default": (None, [C.POINTER(OrcDims)]),
        "orc_load_config": (I, [C.c_char_p, C.POINTER(OrcDims)]),
        "orc_gdn_core": (None, [C.POINTER(OrcDims)] + [P] * 12),
        "orc_attn_core": (None, [C.POINTER(OrcDims), I] + [P] * 8),
        "orc_attn_core_ex": (None, [C.POINTER(OrcDims), I] + [P] * 8 + [I, I]),
        "orc_round_bf16": (F, [F]),
        "orc_round_bf16_array": (None, [P, C.c_int64]),
        "orc_set_kv_bf16": (None, [P, I]),
        "orc_set_prefill_handoff": (None, [P, I]),
        "orc_open": (P, [C.c_char_p, I]),
        "orc_close": (None, [P]),
        "orc_error": (C.c_char_p, []),
        "orc_get_dims": (None, [P, C.POINTER(OrcDims)]),
        "orc_reset": (None, [P]),
        "orc_step": (I, [P, I, P]),
        "orc_generate_greedy": (I, [P, P, I, I, P]),
        "orc_prefill": (I, [P, P, I, P]),
        "orc_position": (I, [P]),
        "orc_set_position": (None, [P, I]),
        "orc_set_trace": (None, [P, P]),
        "orc_hidden": (C.POINTER(C.c_float), [P]),
        "orc_gdn_state": (C.POINTER(C.c_float), [P, I]),
        "orc_conv_state": (C.POINTER(C.c_float), [P, I]),
        "orc_kcache": (C.POINTER(C.c_float), [P, I]),
        "orc_vcache": (C.POINTER(C.c_float), [P, I]),
        "orc_weight_bf16": (C.POINTER(C.c_uint16), [P, C.c_char_p]),
        "orc_weight_f32": (C.POINTER(C.c_float), [P, C.c_char_p]),
        "orc_threads": (I, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


olib = _load_oracle()


def dims_from(d) -> OrcDims:
    """OrcDims from any object with the q35_dims field names (e.g. pyq35.Dims)."""
    o = OrcDims()
    for k, _ in OrcDims._fields_:
        setattr(o, k, getattr(d, k))
    return o


def view(ptr, shape):
    n = int(np.prod(shape))
    return np.ctypeslib.as_array(ptr, shape=(n,)).reshape(shape)


class Oracle:
    """The CPU restatement of QwenModel / QwenForward on a checkpoint directory."""

    def __init__(self, model_dir: str, max_context: int, kv_bf16: bool = False):
        self.h = olib.orc_open(model_dir.encode(), max_context)
        if not self.h:
            raise RuntimeError(f"oracle open failed: {olib.orc_error().decode()}")
        olib.orc_set_kv_bf16(self.h, int(kv_bf16))
        d = OrcDims()
        olib.orc_get_dims(self.h, C.byref(d))
        self.dims = d
        self.max_context = max_context
        self._trace = None

    def close(self):
        if self.h:
            olib.orc_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        olib.orc_reset(self.h)

    def step(self, token: int) -> np.ndarray:
        lg = np.zeros(self.dims.vocab_size, np.float32)
        if olib.orc_step(self.h, int(token), _p(lg)) != 0:
            raise RuntimeError(olib.orc_error().decode())
        return lg

    def generate_greedy(self, prompt, n_new: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        if olib.orc_generate_greedy(self.h, _p(pr), len(pr), n_new, _p(out)) != 0:
            raise RuntimeError(olib.orc_error().decode())
        return out[:n_new]

    def prefill(self, ids, rows: int | None = None, want_logits: bool = True):
        ids = np.ascontiguousarray(ids, np.int32)
        vocab = rows or self.dims.vocab_size
        lg = np.zeros((len(ids), vocab), np.float32) if want_logits else None
        if olib.orc_prefill(self.h, _p(ids), len(ids), _p(lg) if want_logits else None) != 0:
            raise RuntimeError(olib.orc_error().decode())
        return lg

    def set_prefill_handoff(self, on: bool):
        """prefill() leaves its final state in the model, as token-serial steps would."""
        olib.orc_set_prefill_handoff(self.h, int(on))

    def enable_trace(self, rows: int = 1):
        self._trace = np.zeros((rows, self.dims.n_layers_total, self.dims.hidden_size), np.float32)
        olib.orc_set_trace(self.h, _p(self._trace))
        return self._trace

    @property
    def position(self):
        return olib.orc_position(self.h)

    def set_position(self, p):
        olib.orc_set_position(self.h, p)

    def hidden(self):
        return view(olib.orc_hidden(self.h), (self.dims.hidden_size,)).copy()

    def gdn_state(self, i):
        d = self.dims
        return view(olib.orc_gdn_state(self.h, i), (d.gdn_v_heads, d.gdn_k_head_dim, d.gdn_v_head_dim))

    def conv_state(self, i):
        d = self.dims
        conv = 2 * d.gdn_k_heads * d.gdn_k_head_dim + d.gdn_v_heads * d.gdn_v_head_dim
        return view(olib.orc_conv_state(self.h, i), (conv, d.gdn_conv_kernel - 1))

    def kcache(self, i):
        d = self.dims
        return view(olib.orc_kcache(self.h, i), (self.max_context, d.attn_kv_heads, d.attn_head_dim))

    def vcache(self, i):
        d = self.dims
        return view(olib.orc_vcache(self.h, i), (self.max_context, d.attn_kv_heads, d.attn_head_dim))

    def weight_f32(self, name: str, shape) -> np.ndarray:
        p = olib.orc_weight_f32(self.h, name.encode())
        if not p:
            raise KeyError(name)
        return view(p, shape).copy()

    def weight_bf16(self, name: str, shape) -> np.ndarray:
        p = olib.orc_weight_bf16(self.h, name.encode())
        if not p:
            raise KeyError(name)
        return view(p, shape).copy()


def gdn_core(dims, qkv, z, b, a, conv_w, A_log, dt_bias, norm_w, conv_win, S):
    """orc_gdn_core on numpy arrays; conv_win and S are updated in place.
    Returns (raw readout, gated-norm output)."""
    d = dims_from(dims)
    vd = d.gdn_v_heads * d.gdn_v_head_dim
    raw = np.zeros(vd, np.float32)
    out = np.zeros(vd, np.float32)
    args = [np.ascontiguousarray(x, np.float32) for x in (qkv, z, b, a, conv_w, A_log, dt_bias, norm_w)]
    assert conv_win.dtype == np.float32 and conv_win.flags.c_contiguous
    assert S.dtype == np.float32 and S.flags.c_contiguous
    olib.orc_gdn_core(C.byref(d), *[_p(x) for x in args], _p(conv_win), _p(S), _p(raw), _p(out))
    return raw, out


def attn_core(dims, pos, qg, k_new, v_new, q_norm, k_norm, kcache, vcache):
    """orc_attn_core; kcache / vcache [max][NKV][HD] are updated at row pos."""
    d = dims_from(dims)
    out = np.zeros(d.attn_q_heads * d.attn_head_dim, np.float32)
    args = [np.ascontiguousarray(x, np.float32) for x in (qg, k_new, v_new, q_norm, k_norm)]
    assert kcache.dtype == np.float32 and kcache.flags.c_contiguous
    olib.orc_attn_core(C.byref(d), int(pos), *[_p(x) for x in args], _p(kcache), _p(vcache), _p(out))
    return out


def attn_core_ex(dims, pos, qg, k_new, v_new, q_norm, k_norm, kcache, vcache, kv_bf16, append):
    """orc_attn_core_ex: kv_bf16 rounds the appended rows to bf16; append=False attends over
    the caches as given (row pos included)."""
    d = dims_from(dims)
    out = np.zeros(d.attn_q_heads * d.attn_head_dim, np.float32)
    args = [np.ascontiguousarray(x, np.float32) for x in (qg, k_new, v_new, q_norm, k_norm)]
    assert kcache.dtype == np.float32 and kcache.flags.c_contiguous
    assert vcache.dtype == np.float32 and vcache.flags.c_contiguous
    olib.orc_attn_core_ex(C.byref(d), int(pos), *[_p(x) for x in args], _p(kcache), _p(vcache), _p(out),
                          int(kv_bf16), int(append))
    return out


def round_bf16(x):
    """orc_round_bf16_array on a copy: nearest bf16 value (ties to even), as fp32."""
    y = np.array(x, np.float32, copy=True)
    olib.orc_round_bf16_array(_p(y), y.size)
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.zeros_like(x)
    olib.orc_rmsnorm(_p(x), _p(w), _p(y), x.size, eps)
    return y


def rmsnorm_gated(x, w, g, eps):
    x, w, g = (np.ascontiguousarray(v, np.float32) for v in (x, w, g))
    y = np.zeros_like(x)
    olib.orc_rmsnorm_gated(_p(x), _p(w), _p(g), _p(y), x.size, eps)
    return y


def l2norm(x, eps):
    x = np.array(x, np.float32, copy=True)
    olib.orc_l2norm(_p(x), x.size, eps)
    return x


def apply_rope(x, rot, pos, theta):
    x = np.array(x, np.float32, copy=True)
    olib.orc_apply_rope(_p(x), rot, pos, theta)
    return x


def matmul_bf16(W, x):
    W = np.ascontiguousarray(W, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(W.shape[0], np.float32)
    olib.orc_matmul_bf16(_p(W), _p(x), _p(y), W.shape[0], W.shape[1])
    return y


def threads() -> int:
    return olib.orc_threads()


# ----------------------------------------------------------------------------- reference
def ref_available() -> bool:
    return os.path.exists(REF_PATH)


class Ref:
    """The reference engine (unmodified sources) through oracle/ref_harness.cpp."""

    _lib = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            lib = C.CDLL(REF_PATH)
            P, I, F, D = C.c_void_p, C.c_int, C.c_float, C.c_double
            sig = {
                "ref_open": (P, [C.c_char_p, I, I]), "ref_close": (None, [P]),
                "ref_reset": (None, [P]), "ref_position": (I, [P]),
                "ref_set_position": (None, [P, I]), "ref_vocab": (I, [P]),
                "ref_hidden_size": (I, [P]), "ref_step": (I, [P, I, P]),
                "ref_generate_greedy": (I, [P, P, I, I, P]),
                "ref_hidden": (C.POINTER(C.c_float), [P]),
                "ref_normed": (C.POINTER(C.c_float), [P]),
                "ref_gdn_state": (C.POINTER(C.c_float), [P, I]),
                "ref_conv_state": (C.POINTER(C.c_float), [P, I]),
                "ref_kcache": (C.POINTER(C.c_float), [P, I]),
                "ref_vcache": (C.POINTER(C.c_float), [P, I]),
                "ref_mixer": (I, [P, I, P]), "ref_prefill": (I, [P, P, I, P]),
                "ref_rmsnorm": (None, [P, P, P, I, F]),
                "ref_rmsnorm_gated": (None, [P, P, P, P, I, F]),
                "ref_l2norm": (None, [P, I, F]), "ref_apply_rope": (None, [P, I, I, D]),
                "ref_matmul_bf16": (None, [P, P, P, I, I]),
                "ref_budget": (I, [C.c_char_p, I, I, I, P]),
                "ref_solve_max_context": (C.c_int64, [C.c_char_p] + [C.c_uint64] * 6 + [I]),
                "ref_config": (I, [C.c_char_p, P, C.POINTER(C.c_double), C.POINTER(C.c_float),
                                   C.POINTER(C.c_float)]),
            }
            for name, (res, args) in sig.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            cls._lib = lib
        return cls._lib

    def __init__(self, model_dir: str, max_context: int, n_layers: int = 0):
        lib = self.lib()
        self.h = lib.ref_open(model_dir.encode(), max_context, n_layers)
        if not self.h:
            raise RuntimeError("reference open failed")
        self.vocab = lib.ref_vocab(self.h)
        self.H = lib.ref_hidden_size(self.h)

    def close(self):
        if self.h:
            self.lib().ref_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def step(self, token):
        lg = np.zeros(self.vocab, np.float32)
        self.lib().ref_step(self.h, int(token), _p(lg))
        return lg

    def generate_greedy(self, prompt, n_new):
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        self.lib().ref_generate_greedy(self.h, _p(pr), len(pr), n_new, _p(out))
        return out[:n_new]

    def hidden(self):
        return view(self.lib().ref_hidden(self.h), (self.H,)).copy()

    def prefill(self, ids) -> np.ndarray:
        """QwenForward::prefill: logits of every row, [n][vocab]."""
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.zeros((len(ids), self.vocab), np.float32)
        if self.lib().ref_prefill(self.h, _p(ids), len(ids), _p(lg)) != 0:
            raise RuntimeError("reference prefill failed")
        return lg
