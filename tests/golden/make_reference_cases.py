"""Writes reference_unit_cases.json: the inputs and expected results that the
reference's own unit tests hold for this path, transcribed as data (the
reference is C++23 and cannot be compiled here; nothing is imported from it).

Sources:
  tests/test_dtype.cpp:7-24        bf16 round trip values and tolerance, specials
  tests/test_ops_cpu.cpp:118-148   RmsNormImpl<CPU> on [[1,2,3,4],[2,4,6,8]], gamma 1, eps 1e-5
  tests/test_page_attention.cpp:4-85  BlockPool / PagedAttentionManager sequences
  tests/test_tensor.cpp:72-76      Device enum values
Run: python tests/golden/make_reference_cases.py
"""
import json
import math
import os

cases = {
    "bf16_roundtrip": {
        "source": "tests/test_dtype.cpp:7-15",
        "values": [0.0, 1.0, -1.0, 3.140625, 0.5, 65504.0, -65504.0],
        "tolerance": "abs(v) * 1e-2 + 1e-6",
    },
    "bf16_special": {
        "source": "tests/test_dtype.cpp:17-24, include/utils/bfloat16.hpp:114-122",
        "zero_bits": 0,
        "infinity_bits": 0x7F80,
        "neg_infinity_bits": 0xFF80,
        "nan_bits": 0x7FC0,
    },
    "rms_norm": {
        "source": "tests/test_ops_cpu.cpp:118-148",
        "x": [[1.0, 2.0, 3.0, 4.0], [2.0, 4.0, 6.0, 8.0]],
        "gamma": [1.0, 1.0, 1.0, 1.0],
        "eps": 1e-5,
        "checks": [
            {"index": 0, "expected": 1.0 / math.sqrt((1 + 4 + 9 + 16) / 4.0)},
            {"index": 3, "expected": 4.0 / math.sqrt((1 + 4 + 9 + 16) / 4.0)},
            {"index": 4, "expected": 2.0 / math.sqrt((4 + 16 + 36 + 64) / 4.0)},
        ],
        "tolerance": 1e-2,
    },
    "block_pool_alloc_free": {
        "source": "tests/test_page_attention.cpp:4-25",
        "capacity": 100,
        "steps": [["num_blocks", 0], ["num_free", 0], ["alloc", 0], ["num_blocks", 1], ["num_free", 0],
                  ["alloc", 1], ["free", 0], ["num_free", 1], ["alloc", 0], ["num_free", 0]],
    },
    "block_pool_many_allocs": {
        "source": "tests/test_page_attention.cpp:27-35",
        "capacity": 10,
        "allocs_ok": 10,
        "then": -1,
    },
    "block_pool_reset": {
        "source": "tests/test_page_attention.cpp:37-47",
        "capacity": 10,
        "allocs": 3,
        "after_reset": {"num_blocks": 3, "num_free": 3},
        "note": "free list [0,1,2] after reset, so the next alloc pops 2 (comment at :44)",
        "next_alloc": 2,
    },
    "page_table_append_kv": {
        "source": "tests/test_page_attention.cpp:49-64",
        "layer": [0, 8, 128, "BF16"],
        "appends": [[1, 1, None], [31, 32, 2]],
    },
    "page_table_multi_layer": {
        "source": "tests/test_page_attention.cpp:66-85",
        "layers": [[0, 8, 128, "F16"], [1, 4, 64, "F32"]],
        "inactive_layer": 2,
        "appends": [[0, 5], [1, 20]],
        "after_reset": {"layer0_num_cached": 0, "layer1_pages": 0},
    },
    "device_enum": {"source": "tests/test_tensor.cpp:72-76", "CPU": 0, "CUDA": 1, "VULKAN": 4},
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_unit_cases.json")
    with open(out, "w") as f:
        json.dump(cases, f, indent=1)
    print("wrote", out)
