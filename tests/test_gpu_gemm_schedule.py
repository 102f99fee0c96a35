"""GPU parity of the expert GEMMs' work schedule on 256-row tiles.

The up GEMM on 256-row tiles with an even n-tile count pairs an expert's last
M tile of at most 128 rows with two n-tiles (one work item), and the items of
the last, partial round of workgroups (one per CU) are split into K ranges
whose fp32 partials fold_up_kernel sums before the epilogue.  These cases are
built so that both happen, checked against the oracle (layer) or an fp64
product (one expert), within the north-star tolerances (2e-2 bf16, 5e-2 fp8
weights).
"""
import numpy as np
import pytest

from test_gpu_layer import TOL, Case, check_case, rel_err
from test_gpu_stages import _bf16_round

pytestmark = pytest.mark.gpu


def _up_items(counts, n_tiles, bm=256):
    """Work items of the up GEMM: per expert n_tiles times its M tiles, with a
    last M tile of at most bm / 2 rows serving two n-tiles in one item."""
    w, paired = 0, 0
    for c in counts:
        f, r = divmod(int(c), bm)
        if 0 < r <= bm // 2:
            w += n_tiles * f + n_tiles // 2
            paired += 1
        else:
            w += n_tiles * (f + (1 if r else 0))
    return w, paired


@pytest.mark.parametrize("etype,act,wdtype,H", [
    ("gated", "silu", "bf16", 1024),
    ("gated", "silu", "fp8", 1024),
    ("standard", "gelu", "bf16", 2048),
])
def test_paired_items_and_up_tail_split(moe, oracle, etype, act, wdtype, H):
    import torch

    # 16 experts averaging 512 rows: 256-row tiles; a skewed router bias
    # spreads the counts so that several experts end in a tile of <= 128
    # rows; D = 256 gives 8 K stages (split into 4 ranges of 2)
    rng = np.random.default_rng(81)
    bias = (rng.standard_normal(16) * 0.6).astype(np.float32)
    c = Case(moe, oracle, T=4096, D=256, H=H, E=16, k=2, gate="topk", expert_type=etype, act=act,
             wdtype=wdtype, xdtype="bf16", seed=81, router_bias=bias)
    try:
        _, loss, res = c.run(training=True)
        n_tiles = H // (128 if etype == "gated" else 256)
        w, paired = _up_items(res["counts"], n_tiles)
        ncu = torch.cuda.get_device_properties(0).multi_processor_count
        print(f"up items {w} (paired {paired} experts) on {ncu} CUs", flush=True)
        assert paired > 0, "the case must hold paired items"
        assert w > ncu and w % ncu != 0 and 2 * (w % ncu) <= ncu, "the case must split a partial last round"
        check_case(c, TOL[wdtype])
    finally:
        c.dev.close()


@pytest.mark.parametrize("n", [100, 300, 700])
def test_expert_forward_paired_and_split(moe, oracle, n):
    # one expert's rows on a 256-row-tile handle: n = 100 is a single paired
    # item per n-tile pair, 300 = one full tile + a paired item, 700 = two
    # full tiles + a 188-row tile (no pairing); every item of such a small
    # list is split into K ranges and folded
    c = Case(moe, oracle, T=4096, D=256, H=1024, E=16, k=2, wdtype="bf16", xdtype="bf16", seed=82)
    try:
        x = np.ascontiguousarray(c.x[:n])
        print(f"expert_forward 256-row tiles n={n}", flush=True)
        y = c.dev.expert_forward(5, x)
        ex = c.ex[5]
        xd = x.astype(np.float64)
        g = xd @ ex["w1"].T.astype(np.float64)
        u = xd @ ex["w3"].T.astype(np.float64)
        h = _bf16_round(oracle, (g / (1.0 + np.exp(-g))) * u).astype(np.float64)
        ref = h @ ex["w2"].T.astype(np.float64)
        err = rel_err(y, ref)
        assert err <= TOL["bf16"], f"relative error {err:.3e}"
        y2 = c.dev.expert_forward(5, x)
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    finally:
        c.dev.close()
