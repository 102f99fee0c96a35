"""Resources of the built kernels (mixtureofexperts_amd/kernel_resources.json,
written by mixtureofexperts_amd/build.py from the compiler's
kernel-resource-usage remarks of the device pass).

No kernel keeps anything in private (scratch) memory: a register array
indexed at run time, or registers spilled to memory, puts per-lane memory
traffic into a kernel's critical path (a decode routing loop that picked its
part of the experts at run time took the decode up kernel from 6.9 to 19 us).
Every workgroup's LDS fits a CU's 160 KB."""
import json
import os

import pytest

PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mixtureofexperts_amd",
                    "kernel_resources.json")


def _kernels():
    if not os.path.exists(PATH):
        pytest.skip("no kernel_resources.json: the library was not built by mixtureofexperts_amd/build.py here")
    with open(PATH) as f:
        res = json.load(f)
    return {name: v for per_file in res.values() for name, v in per_file.items()}


def test_every_source_reports_its_kernels():
    with open(PATH) if os.path.exists(PATH) else open(os.devnull) as f:
        text = f.read()
    if not text:
        pytest.skip("no kernel_resources.json")
    res = json.loads(text)
    assert set(res) == {"moe_api.hip", "moe_route.hip", "moe_gemm.hip", "moe_gemm_bf16.hip", "moe_decode.hip"}
    assert all(len(v) > 0 for v in res.values())


def test_no_kernel_uses_private_memory():
    k = _kernels()
    bad = {name: v["scratch"] for name, v in k.items() if v.get("scratch", 0) > 0}
    assert not bad, bad
    spills = {name: v["vgpr_spill"] for name, v in k.items() if v.get("vgpr_spill", 0) > 0}
    assert not spills, spills


def test_lds_fits_a_cu():
    k = _kernels()
    big = {name: v["lds"] for name, v in k.items() if v.get("lds", 0) > 160 * 1024}
    assert not big, big
