"""The allocation-free decode entry point (genllm_paged_decode_noalloc) against
the entry point it mirrors (genllm_paged_decode with a caller workspace): the
same kernels and split plan, so the outputs must be bit-identical, on two calls
in a row -- the second with a smaller input -- and after a call that needs more
than the fixed scratch, which must be refused without launching anything.
Also checked against the oracle to the attention tolerance."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import ERR_INVALID, GenllmError
from helpers import assert_attn_close, oracle_fragmented, scale_for

pytestmark = pytest.mark.gpu

SCRATCH = 4 << 20


class Cache:
    def __init__(self, orc, Hkv, D, pool, n_ctx, seed):
        perm_k, perm_v = synth.shuffled(seed, pool), synth.shuffled(seed + 1, pool)
        self.mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2)
        self.mgr.init_layer(0, Hkv, D)
        self.mgr.reserve_layer(0, pool)
        self.mgr.fragment(0, perm_k, perm_v)
        self.mgr.append_kv_pages(0, n_ctx)
        self.ref = oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v)
        self.ref.append_kv_pages(0, n_ctx)
        kp = synth.normal_bf16(seed + 2, (pool, 16, Hkv, D))
        vp = synth.normal_bf16(seed + 3, (pool, 16, Hkv, D))
        self.ref.pool_array(0, 0)[:] = kp
        self.ref.pool_array(0, 1)[:] = vp
        self.mgr.write_pool(0, 0, kp)
        self.mgr.write_pool(0, 1, vp)
        self.info = self.mgr.get_layer(0)
        self.Hkv, self.D, self.n_ctx = Hkv, D, n_ctx

    def run(self, q_bits, n_cached, noalloc):
        Hq, S, D = q_bits.shape
        out = torch.zeros((Hq, S, D), dtype=torch.bfloat16, device="cuda")
        n_pages = (n_cached + 15) // 16
        i = self.info
        q = paged.to_device_bf16(q_bits)
        print(f"decode {'noalloc' if noalloc else 'workspace'}: Hq={Hq} S={S} D={D} n_cached={n_cached}", flush=True)
        if noalloc:
            paged.paged_decode_noalloc(q, out, i.k_pool, i.v_pool, i.k_ids, i.v_ids, n_pages, n_cached, self.Hkv,
                                       scale_for(D))
        else:
            ws = torch.zeros(paged.decode_workspace_bytes(Hq, self.Hkv, S, D, n_pages), dtype=torch.uint8,
                             device="cuda")
            paged.paged_decode(q, out, i.k_pool, i.v_pool, i.k_ids, i.v_ids, n_pages, n_cached, self.Hkv,
                               scale_for(D), ws)
        torch.cuda.synchronize()
        return paged.to_host_bits(out)

    def oracle(self, q_bits):
        Hq, S, D = q_bits.shape
        out, rc = self.ref.paged_attend(0, q_bits[None], self.Hkv, Hq // self.Hkv, scale_for(D), True)
        assert rc == 0
        return out[0]

    def close(self):
        self.mgr.close()


@pytest.mark.parametrize("merge", ["kernel", "kernel", "fused"])
def test_noalloc_matches_workspace_entry_point(orc, merge, request):
    paged.decode_tuning(0, merge)
    request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    # config 3's shape (8193 keys, 32 q / 8 kv heads), then a smaller call on
    # the same scratch: fewer keys, fewer rows
    c = Cache(orc, 8, 128, 600, 8193, 4242)
    q1 = synth.normal_bf16(4243, (32, 1, 128))
    a = c.run(q1, 8193, noalloc=True)
    b = c.run(q1, 8193, noalloc=False)
    assert np.array_equal(a, b), "noalloc differs from the workspace entry point (8193 keys)"
    assert_attn_close(a, c.oracle(q1), "noalloc 8193 keys")
    c.close()
    c2 = Cache(orc, 8, 128, 40, 517, 4244)
    q2 = synth.normal_bf16(4245, (16, 1, 128))
    a2 = c2.run(q2, 517, noalloc=True)
    b2 = c2.run(q2, 517, noalloc=False)
    assert np.array_equal(a2, b2), "noalloc differs from the workspace entry point (517 keys, 2nd call)"
    assert_attn_close(a2, c2.oracle(q2), "noalloc 517 keys")
    c2.close()


def test_noalloc_long_context_four_heads(orc):
    """At config 5's length (32,761 keys) the plan reads 4 kv heads per split
    workgroup over 128 splits (2.1 MiB of partials, inside the scratch): the
    allocation-free call matches the workspace call bit for bit, and the
    oracle to the attention tolerance; then a shorter call (one-head plan)."""
    c = Cache(orc, 8, 128, 2060, 32761, 0x5EED0905)
    q1 = synth.normal_bf16(0x5EED0906, (32, 1, 128))
    a = c.run(q1, 32761, noalloc=True)
    b = c.run(q1, 32761, noalloc=False)
    assert np.array_equal(a, b), "noalloc differs from the workspace entry point (32761 keys)"
    assert_attn_close(a, c.oracle(q1), "noalloc 32761 keys")
    a2 = c.run(q1, 8193, noalloc=True)
    b2 = c.run(q1, 8193, noalloc=False)
    assert np.array_equal(a2, b2), "noalloc differs from the workspace entry point (8193 keys after 32761)"
    c.close()


def test_noalloc_refuses_plans_beyond_its_scratch(orc, request):
    """16 rows per kv head over 8 kv heads at 8193 keys with 3 pages per
    split: 8 x 171 splits x 16 rows x 130 x 4 B = 11.4 MB of partials, more
    than the 4 MiB scratch -- refused with GENLLM_ERR_INVALID, output
    untouched; the next call that fits still matches the workspace entry
    point."""
    paged.decode_tuning(3, "kernel")
    request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    c = Cache(orc, 8, 128, 600, 8193, 4246)
    q = paged.to_device_bf16(synth.normal_bf16(4247, (32, 4, 128)))  # G=4, S=4: 16 rows
    out = torch.zeros((32, 4, 128), dtype=torch.bfloat16, device="cuda")
    i = c.info
    with pytest.raises(GenllmError) as e:
        paged.paged_decode_noalloc(q, out, i.k_pool, i.v_pool, i.k_ids, i.v_ids, 513, 8193, 8, scale_for(128))
    assert e.value.code == ERR_INVALID and "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert not out.float().abs().sum().item()
    paged.decode_tuning(0, "kernel")
    q1 = synth.normal_bf16(4248, (32, 1, 128))
    assert np.array_equal(c.run(q1, 8193, noalloc=True), c.run(q1, 8193, noalloc=False))
    c.close()


def test_noalloc_first_call_under_capture():
    """The first call on a device resolves its scratch (hipGetSymbolAddress)
    and clears the counters with a kernel on the caller's stream; made while
    a HIP graph is being captured (a fresh process, so it really is the
    first), the graph's replays equal the workspace entry point bit for bit
    (tests/noalloc_capture_child.py)."""
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_child.py")
    r = subprocess.run([sys.executable, child], capture_output=True, text=True, timeout=150)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
