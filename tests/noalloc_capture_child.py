"""Child process of test_zz_no_alloc.test_noalloc_first_call_under_capture:
the first genllm_paged_decode_noalloc call of a fresh process (the one that
resolves the device's scratch and clears its counters) made while a HIP graph
is being captured.  Each replay, with eager work on the stream between
replays, must equal the workspace entry point bit for bit.  Prints CAPTURE_OK."""
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from genllm_amd import paged, synth  # noqa: E402
from helpers import scale_for  # noqa: E402

Hq, Hkv, D, pool, n_ctx = 32, 8, 128, 600, 8193
torch.cuda.set_device(0)
mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2)
mgr.init_layer(0, Hkv, D)
mgr.reserve_layer(0, pool)
mgr.fragment(0, synth.shuffled(77, pool), synth.shuffled(78, pool))
mgr.append_kv_pages(0, n_ctx)
mgr.write_pool(0, 0, synth.normal_bf16(79, (pool, 16, Hkv, D)))
mgr.write_pool(0, 1, synth.normal_bf16(80, (pool, 16, Hkv, D)))
i = mgr.get_layer(0)
n_pages = (n_ctx + 15) // 16
q = torch.empty((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
out_g = torch.zeros((Hq, 1, D), dtype=torch.bfloat16, device="cuda")
out_w = torch.zeros_like(out_g)
ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, n_pages), dtype=torch.uint8, device="cuda")
torch.cuda.synchronize()
print("capturing the first noalloc call of this process", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    paged.paged_decode_noalloc(q, out_g, i.k_pool, i.v_pool, i.k_ids, i.v_ids, n_pages, n_ctx, Hkv, scale_for(D))
for rep in range(3):
    paged.fill_normal_bf16(q, 100 + rep)
    out_g.zero_()
    g.replay()
    paged.paged_decode(q, out_w, i.k_pool, i.v_pool, i.k_ids, i.v_ids, n_pages, n_ctx, Hkv, scale_for(D), ws)
    torch.cuda.synchronize()
    a, b = paged.to_host_bits(out_g), paged.to_host_bits(out_w)
    assert np.array_equal(a, b), f"replay {rep}: captured noalloc decode differs from the workspace entry point"
    assert np.any(a != 0), f"replay {rep}: no output"
    print(f"replay {rep} matches", flush=True)
del g
mgr.close()
print("CAPTURE_OK", flush=True)
