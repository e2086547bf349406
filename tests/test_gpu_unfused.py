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
        _native.EPI_BIAS_LEAKY: (True, "leaky"), _native.EPI_NONE: (False, "none"),
        _native.EPI_BIAS_IF_RELU: (True, "if_relu"), _native.EPI_IF_RELU: (False, "if_relu")}


@pytest.mark.parametrize("M, K, N", [(1024, 1024, 1024), (16, 8192, 1024), (129, 77, 131), (1, 64, 5)])
@pytest.mark.parametrize("epi", sorted(_ACT))
@pytest.mark.parametrize("bias_offset", [0, 1], ids=["bias-aligned", "bias-misaligned"])
def test_unfused_sequence_equals_the_fused_launch(M, K, N, epi, bias_offset):
    """With the bias one element off 16-byte alignment the fused launch
    takes kernels for unaligned operands; the unfused sequence's GEMM plans
    with that bias too, so both still run the same kernel."""
    import torch
    rng = np.random.default_rng(M * 7 + K + N + epi)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    tX, tW = (torch.from_numpy(a).cuda() for a in (X, W))
    tb = torch.zeros(N + bias_offset, device="cuda")[bias_offset:]
    tb.copy_(torch.from_numpy(b))
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
    assert plans[1].split(" | ")[1] == plans[0], plans  # the same GEMM kernel
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    bias, act = _ACT[epi]
    assert_f32_parity(outs[1], oracle.dense_f32_chains(X, W, b if bias else None, act, 0.03), K)
