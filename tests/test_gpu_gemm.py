"""GPU parity of spinn_hip_gemm (Gemm / MatMul) against the oracle and float64."""
import numpy as np
import pytest

from oracle import oracle as O
from spinn_amd.models import GEMM_SWEEP
from tests.conftest import assert_parity
from tests.hipops import run_gemm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mnk", GEMM_SWEEP, ids=[f"{m}x{n}x{k}" for m, n, k in GEMM_SWEEP])
def test_gemm_sweep(hip, torch_gpu, mnk):
    """The Gemm sweep: A ~ U(-1,1) [M,K], B ~ N(0,1/K) [N,K] (transB=1), bias ~ N(0,0.01) [N]."""
    m, n, k = mnk
    print(f"[gemm] {mnk}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    c = rng.normal(0, 0.01, n).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, c, trans_b=1)
    assert_parity(y, O.gemm(a, b, c, trans_b=1), what="vs oracle")
    assert_parity(y, O.gemm_f64(a, b, c, trans_b=1), what="vs float64")


@pytest.mark.parametrize("m", [37, 19], ids=["m37", "m19_32row_tile"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("cmode", [0, 1, 2])
def test_gemm_transposes_ragged(hip, torch_gpu, ta, tb, cmode, m):
    n, k = 45, 29
    rng = np.random.default_rng(100 + 4 * ta + 2 * tb + cmode + m)
    a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    c = None if cmode == 0 else rng.uniform(-1, 1, n if cmode == 1 else (m, n)).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb)
    assert_parity(y, O.gemm_f64(a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb), what="vs float64")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [2048, 2047, 600, 5], ids=["k2048", "k2047_scalar", "k600", "k5"])
@pytest.mark.parametrize("cmode", [0, 1, 2])
def test_gemm_few_rows_fc(hip, torch_gpu, m, k, cmode):
    """M <= 4 with transB=1 (fully-connected layers) runs waves over the rows of B: one per
    output column below K = 1024, else two (M = 1) or four (M > 1), each summing its share of
    K; float4 loads when K % 4 == 0, scalar otherwise; alpha, beta and both C forms; 999
    columns leave the last workgroup part-filled."""
    n = 1000 if k == 2048 else 999
    rng = np.random.default_rng(m * 10 + k + cmode)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    c = None if cmode == 0 else rng.uniform(-1, 1, n if cmode == 1 else (m, n)).astype(np.float32)
    print(f"[gemm] fc m={m} k={k} cmode={cmode}", flush=True)
    y = run_gemm(hip, torch_gpu, a, b, c, alpha=0.75, beta=1.5, trans_b=1)
    assert_parity(y, O.gemm_f64(a, b, c, alpha=0.75, beta=1.5, trans_b=1), what="vs float64")


def test_gemm_aligned_large(hip, torch_gpu):
    m, n, k = 512, 768, 1024
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b)
    assert_parity(y, O.gemm(a, b, None, beta=0.0), what="vs oracle")


def test_matmul_batched(hip, torch_gpu):
    bt, m, n, k = 3, 33, 40, 20
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, (bt, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (bt, k, n)).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, alpha=1.0, beta=0.0, batch=bt)
    assert_parity(y, O.matmul(a, b), what="vs oracle")
