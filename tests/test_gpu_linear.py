"""GPU parity of genllm_linear (LinearImpl: linear.cpp:46-122, linear.cu:72-126)
against the CPU oracle's restatement of the reference's bf16 linear.

rows <= 4 (the decode GEMV): the kernel follows the reference's summation
order, so outputs are compared bit for bit.  More rows go through rocBLAS (its
own summation order): within one bf16 rounding plus fp32 accumulation error of
the fp64 result, and mostly bit-equal to the oracle."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import GenllmError, call

pytestmark = pytest.mark.gpu


def bits_dev(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda()


def run_linear(x, w, bias=None):
    rows, common = x.shape
    cols = w.shape[0]
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda")
    need = paged.linear_workspace_bytes(rows, common, cols)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda") if need else None
    paged.linear(bits_dev(x), bits_dev(w), out, None if bias is None else bits_dev(bias), ws)
    torch.cuda.synchronize()
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


def inputs(seed, rows, common, cols, wscale=0.05):
    rng = np.random.default_rng(seed)
    x = synth.f32_to_bf16_bits(rng.standard_normal((rows, common)).astype(np.float32))
    w = synth.f32_to_bf16_bits((rng.standard_normal((cols, common)) * wscale).astype(np.float32))
    b = synth.f32_to_bf16_bits(rng.standard_normal(cols).astype(np.float32))
    return x, w, b


@pytest.mark.parametrize("rows,common,cols", [
    (1, 2560, 6144),   # Qwen3-4B fused QKV projection of one decode token
    (1, 1024, 4096),   # Qwen3-0.6B
    (2, 256, 300),
    (3, 264, 77),      # a block with a trailing 8-group
    (4, 520, 129),
    (1, 8, 5),         # one 8-group only
    (4, 24, 1000),
    (1, 32768, 3),     # 128 K-blocks: one column per workgroup
    # whole K-blocks: the LDS-staged kernel (weights and x through LDS)
    (4, 2560, 6144),
    (3, 512, 77),      # the last workgroup holds 13 of its 64 columns
    (2, 1280, 101),    # 5 blocks per column: an odd block count per workgroup (125)
    (1, 4096, 130),
    (1, 8192, 64),     # 80 KB of LDS: the largest staged shape
    (2, 8192, 64),     # 96 KB of LDS: the direct-load kernel
    (1, 768, 97),      # 3 blocks per column: 126 blocks per workgroup, the last 1 KB load of each part half full
    (3, 1792, 50),     # 7 blocks per column: 126 blocks, 3 rows of x
])
def test_linear_gemv_bit_exact(orc, rows, common, cols):
    x, w, b = inputs(rows * 1000 + common + cols, rows, common, cols)
    assert paged.linear_workspace_bytes(rows, common, cols) == 0
    assert np.array_equal(run_linear(x, w), orc.linear(x, w))
    assert np.array_equal(run_linear(x, w, b), orc.linear(x, w, b))


def test_linear_gemv_order_cases(orc):
    # the hand-derived order pins of the oracle test, through the GPU kernel
    common = 512
    x = np.zeros((1, common), dtype=np.float32)
    w = np.zeros((1, common), dtype=np.float32)
    x[0, 0], w[0, 0] = 4096.0, 4096.0
    x[0, 8], w[0, 8] = 1.0, 1.0
    x[0, 24], w[0, 24] = 1.0, 1.0
    x[0, 256], w[0, 256] = 4096.0, -4096.0
    xb, wb = synth.f32_to_bf16_bits(x), synth.f32_to_bf16_bits(w)
    got = run_linear(xb, wb)
    assert synth.bf16_bits_to_f32(got)[0, 0] == 2.0
    assert np.array_equal(got, orc.linear(xb, wb))


@pytest.mark.parametrize("rows,common,cols,with_bias", [
    (5, 2560, 512, True),
    (64, 1024, 1024, True),
    (300, 2560, 640, True),
    (2, 20, 33, True),       # common % 8 != 0 also takes the GEMM path
    (64, 1024, 1024, False),  # no bias: rocBLAS rounds straight into out
    (2048, 2560, 768, False),
])
def test_linear_gemm_within_tolerance(orc, rows, common, cols, with_bias):
    x, w, b = inputs(rows + common + cols, rows, common, cols)
    if not with_bias:
        b = None
    assert paged.linear_workspace_bytes(rows, common, cols) == rows * cols * 4
    got = synth.bf16_bits_to_f32(run_linear(x, w, b)).astype(np.float64)
    want = orc.linear(x, w, b)
    xf, wf = synth.bf16_bits_to_f32(x).astype(np.float64), synth.bf16_bits_to_f32(w).astype(np.float64)
    bf = synth.bf16_bits_to_f32(b).astype(np.float64) if b is not None else np.zeros(cols)
    exact = xf @ wf.T + bf[None, :]
    mag = np.abs(xf) @ np.abs(wf).T + np.abs(bf)[None, :]
    e = np.abs(exact)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(e, 2.0 ** -126))) - 7)
    tol = ulp / 2 + common * 2.0 ** -24 * mag  # one bf16 rounding + fp32 accumulation
    assert np.all(np.abs(got - exact) <= tol)
    same = np.mean(run_linear(x, w, b) == want)
    print(f"gemm rows{rows} common{common} cols{cols}: {same:.4f} of outputs bit-equal to the oracle")
    assert same > 0.9


def test_linear_errors():
    x = torch.zeros((8, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((16, 64), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((8, 16), dtype=torch.bfloat16, device="cuda")
    bias = torch.zeros((16,), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(GenllmError):
        paged.linear(x, w, out, bias=bias)  # 8 rows with a bias need a workspace
    small = torch.empty(8 * 16 * 4 - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(GenllmError):
        paged.linear(x, w, out, bias=bias, workspace=small)
    paged.linear(x, w, out)  # without a bias the GEMM rounds straight into out: no workspace
    with pytest.raises(GenllmError):
        call("genllm_linear", None, w.data_ptr(), None, out.data_ptr(), 1, 64, 16, None, 0, None)
    # zero rows: nothing to do
    call("genllm_linear", x.data_ptr(), w.data_ptr(), None, out.data_ptr(), 0, 64, 16, None, 0, None)
