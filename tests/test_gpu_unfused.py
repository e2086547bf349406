"""The reference's unfused GPU sequence on this library's kernels
(edsl_hip_dense_f32_launch_unfused: fill, GEMM without epilogue, separate
bias + activation pass) equals the fused launch bit for bit, and the oracle
to the fp32 bar. The benchmark times the two side by side."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native

pytestmark = pytest.mark.gpu

_ACT = {_native.EPI_BIAS_RELU: (True, "relu"), _native.EPI_BIAS: (True, "none"), _native.EPI_RELU: (False, "relu"),
        _native.EPI_BIAS_LEAKY: (True, "leaky"), _native.EPI_NONE: (False, "none")}


@pytest.mark.parametrize("M, K, N", [(1024, 1024, 1024), (16, 8192, 1024), (129, 77, 131), (1, 64, 5)])
@pytest.mark.parametrize("epi", sorted(_ACT))
def test_unfused_sequence_equals_the_fused_launch(M, K, N, epi):
    import torch
    rng = np.random.default_rng(M * 7 + K + N + epi)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    tX, tW, tb = (torch.from_numpy(a).cuda() for a in (X, W, b))
    L = _native.lib()
    outs, plans = [], []
    for entry in (L.edsl_hip_dense_f32_launch, L.edsl_hip_dense_f32_launch_unfused):
        tY = torch.full((M, N), float("nan"), device="cuda")
        rc = entry(tX.data_ptr(), K, tW.data_ptr(), N, tb.data_ptr(), tY.data_ptr(), N, M, N, K, epi, 0.03,
                   torch.cuda.current_stream().cuda_stream)
        assert rc == 0, _native.last_error()
        plans.append(_native.last_plan())
        torch.cuda.synchronize()
        outs.append(tY.cpu().numpy())
    assert plans[1].startswith("unfused: fill | ") and plans[1].endswith(f"bias_act epi={epi}"), plans[1]
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    bias, act = _ACT[epi]
    assert_f32_parity(outs[1], oracle.dense_f32_chains(X, W, b if bias else None, act, 0.03), K)
