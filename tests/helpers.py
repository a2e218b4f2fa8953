"""Shared helpers of the test suite."""
from __future__ import annotations

import hashlib
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Parity bars: per-layer hidden states and GDN state within
# rel_l2 <= 1e-5 of the reference CPU fp32 path; greedy ids identical.
REL_L2 = 1e-5


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for blk in iter(lambda: f.read(1 << 24), b""):
            h.update(blk)
    return h.hexdigest()


_gpu = None


def gpu_count() -> int:
    global _gpu
    if _gpu is None:
        try:
            import pyq35

            _gpu = pyq35.Hip().device_count()
        except Exception:
            _gpu = 0
    return _gpu


def ring_from_window(win: np.ndarray, pos: int) -> np.ndarray:
    """Device conv ring [4][CONV] (input of position t in slot t % 4) holding the
    reference window [CONV][3] (inputs of positions pos-3, pos-2, pos-1) at position pos."""
    conv = win.shape[0]
    ring = np.zeros((4, conv), np.float32)
    for k in range(3):
        ring[(pos - 3 + k) % 4] = win[:, k]
    return ring


def window_from_ring(ring: np.ndarray, pos: int) -> np.ndarray:
    """Reference window [CONV][3] at position pos (after `pos` steps) from the device ring."""
    return np.stack([ring[(pos - 3 + k) % 4] for k in range(3)], axis=1)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint32) << 16).view(np.float32)


def read_safetensors(path: str) -> dict:
    """name -> numpy array (BF16 as uint16 bit patterns, F32 as float32)."""
    import json

    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(n))
        base = 8 + n
        out = {}
        for name, e in header.items():
            if name == "__metadata__":
                continue
            dt = {"BF16": np.uint16, "F32": np.float32}[e["dtype"]]
            a, b = e["data_offsets"]
            f.seek(base + a)
            out[name] = np.frombuffer(f.read(b - a), dtype=dt).reshape(e["shape"])
    return out


def conv_dim(d) -> int:
    return 2 * d.gdn_k_heads * d.gdn_k_head_dim + d.gdn_v_heads * d.gdn_v_head_dim


def layer_name(l: int, suffix: str) -> str:
    return f"model.language_model.layers.{l}.{suffix}"
