"""The C++ host side (genllm_amd/host -> libgenllm_ops.so): the reference's
operator interface (Tensor, PagedAttentionManager, ops::*Impl<Device::HIP>,
kernel::dispatch) over the C ABI.

CPU: the library and the C++ test binary are built and export the operator
entry points.  GPU: tests/cpp/test_ops_hip runs every case of the reference's
tests/test_page_attention.cpp through the HIP manager, then the ops (paged
attention over a 2-layer graph, FlashAttention, RMSNorm, RoPE and its
tables) against the CPU oracle."""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OPS_LIB = os.path.join(ROOT, "genllm_amd", "libgenllm_ops.so")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "test_ops_hip")

EXPECTED = [
    "ops::PagedAttentionImpl<(Device)2>::execute(Tensor*, int)",
    "ops::FlashAttentionImpl<(Device)2>::execute(Tensor*, int)",
    "ops::RmsNormImpl<(Device)2>::execute(Tensor*, int)",
    "ops::ApplyRopeImpl<(Device)2>::execute(Tensor*, int)",
    "ops::RopeCacheImpl<(Device)2>::execute(Tensor*, int)",
    "kernel::paged_attention(Tensor*, int)",
    "kernel::flash_attention(Tensor*, int)",
    "kernel::dispatch(Tensor*, int)",
    "PagedAttentionManager::append_kv_from_tensor(int, void const*, void const*, int, int, int, DataType)",
    "PagedAttentionManager::append_kv_pages(int, int)",
]


def test_ops_library_exports_operator_interface():
    assert os.path.exists(OPS_LIB), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-DC", "--defined-only", OPS_LIB], check=True, capture_output=True, text=True).stdout
    missing = [s for s in EXPECTED if s not in out]
    assert not missing, missing


def test_cpp_test_binary_built():
    assert os.path.exists(TEST_BIN) and os.access(TEST_BIN, os.X_OK), "run __graft_entry__.build() first"


@pytest.mark.gpu
def test_cpp_operator_suite():
    print("running", TEST_BIN, flush=True)
    r = subprocess.run([TEST_BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout[-6000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "FAIL" not in r.stdout
