"""The allocation-free entry point moe_switch_loss_noalloc (device buffers,
partials in the library's static device array) against the allocating
moe_switch_loss on the same inputs: bit-identical losses (the same kernels),
and both within the balance-loss bar (1e-5) of the oracle."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _route(oracle, rng, T, E, k):
    lg = rng.standard_normal((T, E)).astype(np.float32)
    idx, _, probs = oracle.compute_gates_topk(lg, k)
    idx[rng.random(idx.shape) < 0.05] = 0  # dropped entries count in the length only
    return np.ascontiguousarray(idx), np.ascontiguousarray(probs)


def test_switch_loss_noalloc_matches_allocating_entry(moe, oracle):
    torch = pytest.importorskip("torch")
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    rng = np.random.default_rng(5150)
    stream = torch.cuda.Stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    # two calls in a row on the shared array, the second with a smaller input
    for T, E, k in ((40000, 128, 2), (3000, 8, 2), (1, 64, 6)):
        print(f"switch loss noalloc T={T} E={E} k={k}", flush=True)
        idx, probs = _route(oracle, rng, T, E, k)
        ref = ctypes.c_float(0.0)
        _lib.check(L.moe_switch_loss(idx.ctypes.data, T, k, probs.ctypes.data, E, ctypes.c_float(0.01),
                                     ctypes.byref(ref)), None)
        di = torch.from_numpy(idx).cuda()
        dp = torch.from_numpy(probs).cuda()
        out = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        _lib.check(L.moe_switch_loss_noalloc(di.data_ptr(), T, k, dp.data_ptr(), E, ctypes.c_float(0.01),
                                             out.data_ptr(), sp), None)
        stream.synchronize()
        got = np.float32(out.item())
        assert got.view(np.uint32) == np.float32(ref.value).view(np.uint32), (got, ref.value)
        want = oracle.switch_loss(idx, probs, 0.01)
        assert abs(got - want) <= 1e-5 * max(1.0, abs(float(want)))


def test_switch_loss_noalloc_limits(moe):
    torch = pytest.importorskip("torch")
    from mixtureofexperts_amd import _lib

    L = _lib.lib()
    out = torch.zeros(1, dtype=torch.float32, device="cuda")
    # more experts than the scratch array holds: a clear error, nothing launched
    st = L.moe_switch_loss_noalloc(None, 4, 1, None, 513, ctypes.c_float(0.01), out.data_ptr(), None)
    assert st == _lib.MOE_EINVAL
    assert "MOE_MAX_EXPERTS" in L.moe_last_error(None).decode()
    # an empty batch: the NaN of a mean over no tokens, as moe_switch_loss returns
    _lib.check(L.moe_switch_loss_noalloc(None, 0, 2, None, 8, ctypes.c_float(0.01), out.data_ptr(), None), None)
    torch.cuda.synchronize()
    assert np.isnan(out.item())
