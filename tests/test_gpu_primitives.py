"""forward_pass.h primitives on the GPU (q35_matmul_bf16, q35_rmsnorm, q35_rmsnorm_gated,
q35_l2norm, q35_apply_rope) against the oracle on the same inputs."""
import numpy as np
import pytest

import oracle_py as op
import pyq35
from helpers import bf16_bits, rel_l2

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(7)


@pytest.fixture(scope="module")
def hip():
    return pyq35.Hip()


@pytest.mark.parametrize("rows,cols", [(1, 8), (5, 8), (64, 2048), (2048, 6144), (8193, 1024),
                                       (300, 520), (17, 4096), (12288, 2048)])
def test_matmul_bf16(hip, rows, cols):
    W = bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32) * 0.02)
    x = rng.standard_normal(cols).astype(np.float32)
    dW, dx, dy = hip.upload(W), hip.upload(x), hip.malloc(rows * 4)
    try:
        pyq35.check(pyq35.lib.q35_matmul_bf16(dW, dx, dy, rows, cols, None))
        hip.sync()
        y = hip.download(dy, rows)
    finally:
        for p in (dW, dx, dy):
            hip.free(p)
    ref = op.matmul_bf16(W, x)
    assert rel_l2(y, ref) < 1e-6
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("rows,n", [(1, 256), (8, 1024), (3, 2048), (5, 4096), (2, 100)])
def test_rmsnorm_and_gated(hip, rows, n):
    eps = 1e-6
    x = rng.standard_normal((rows, n)).astype(np.float32)
    w = (0.1 * rng.standard_normal(n)).astype(np.float32)
    z = rng.standard_normal((rows, n)).astype(np.float32)
    dx, dw, dz, dy = hip.upload(x), hip.upload(w), hip.upload(z), hip.malloc(x.nbytes)
    try:
        pyq35.check(pyq35.lib.q35_rmsnorm(dx, dw, dy, rows, n, eps, None))
        hip.sync()
        y = hip.download(dy, (rows, n))
        pyq35.check(pyq35.lib.q35_rmsnorm_gated(dx, dw, dz, dy, rows, n, eps, None))
        hip.sync()
        yg = hip.download(dy, (rows, n))
    finally:
        for p in (dx, dw, dz, dy):
            hip.free(p)
    for r in range(rows):
        np.testing.assert_allclose(y[r], op.rmsnorm(x[r], w, eps), rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(yg[r], op.rmsnorm_gated(x[r], w, z[r], eps), rtol=5e-6, atol=1e-7)


def test_l2norm_and_rope(hip):
    rows, hd, rot, theta = 6, 256, 64, 1e7
    x = rng.standard_normal((rows, hd)).astype(np.float32)
    pos = np.array([0, 1, 255, 8191, 131071, 262143], np.int32)
    dx, dp = hip.upload(x), hip.upload(pos)
    try:
        pyq35.check(pyq35.lib.q35_l2norm(dx, rows, hd, 1e-6, None))
        hip.sync()
        l2 = hip.download(dx, (rows, hd))
        hip.copy_in(dx, x)
        pyq35.check(pyq35.lib.q35_apply_rope(dx, rows, hd, rot, dp, 0, theta, None))
        hip.sync()
        rp = hip.download(dx, (rows, hd))
    finally:
        hip.free(dx)
        hip.free(dp)
    for r in range(rows):
        np.testing.assert_allclose(l2[r], op.l2norm(x[r], 1e-6), rtol=2e-6, atol=1e-8)
        ref = op.apply_rope(x[r], rot, int(pos[r]), theta)
        # angles in double on both sides: equal up to the fp32 rotation arithmetic
        np.testing.assert_allclose(rp[r], ref, rtol=1e-6, atol=1e-6)
        np.testing.assert_array_equal(rp[r, rot:], x[r, rot:])


def test_forward_pass_dropin_vs_oracle():
    """The forward_pass.h drop-in called from a C++ program built against the header:
    l2norm, both matmul overloads (the matvec, blocks of rows beyond the staging buffer, rows
    wider than the matvec, rows not a multiple of 8, fp32 weights), rmsnorm, rmsnorm_gated and
    apply_rope (odd and full rotary widths) against the oracle, on the GPU."""
    import os
    import subprocess

    caller = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "forward_pass_caller")
    r = subprocess.run([caller], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
