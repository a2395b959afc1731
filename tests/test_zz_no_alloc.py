"""bh_radix_argsort_noalloc: the allocation-free sort against bh_radix_argsort.

Two calls in a row through the C ABI, the second with a smaller input (the
fixed device scratch keeps the first call's contents, so anything that must
start at zero has to be cleared by the call itself), each compared bit for bit
with the pool-backed entry point on the same keys; the context's workspace
pool does not grow during the allocation-free calls; a size beyond the stated
maximum is rejected before any launch.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _keys(n, bits, seed):
    rng = np.random.default_rng(seed)
    keys = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    if bits and bits < 32:
        keys[: n // 2] &= np.uint32((1 << bits) - 1)
    return keys


def _sort(gpu, fn_name, keys, bits):
    import torch
    from brush_amd import _lib

    ctx = _lib.context()
    n = keys.size
    tk = torch.from_numpy(keys.view(np.int32)).to(gpu)
    tv = torch.arange(n, dtype=torch.int32, device=gpu)
    ok = torch.empty_like(tk)
    ov = torch.empty_like(tv)
    torch.cuda.synchronize()
    status = getattr(_lib.lib(), fn_name)(ctx.handle, _lib.ptr(tk), _lib.ptr(tv), n, bits, _lib.ptr(ok), _lib.ptr(ov))
    ctx.check(status, fn_name)
    torch.cuda.synchronize()
    return ok.cpu().numpy().view(np.uint32), ov.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("first,second", [((2_097_152, 20), (150_001, 32)), ((1_000_003, 32), (4097, 13))])
def test_noalloc_sort_matches_the_pool_sort(gpu, first, second):
    from brush_amd import _lib

    ctx = _lib.context()
    for k, (n, bits) in enumerate((first, second)):
        print(f"[case] radix_argsort_noalloc call {k}: n={n} bits={bits}", flush=True)
        keys = _keys(n, bits, 17 * n + bits)
        want_k, want_v = _sort(gpu, "bh_radix_argsort", keys, bits)
        before = ctx.workspace_bytes()
        got_k, got_v = _sort(gpu, "bh_radix_argsort_noalloc", keys, bits)
        assert ctx.workspace_bytes() == before, "the allocation-free sort used the workspace pool"
        assert np.array_equal(got_k, want_k), f"keys differ (n={n}, bits={bits})"
        assert np.array_equal(got_v, want_v), f"values differ (n={n}, bits={bits})"


def test_noalloc_sort_rejects_sizes_beyond_the_scratch(gpu):
    import torch
    from brush_amd import _lib

    print("[case] radix_argsort_noalloc beyond the maximum", flush=True)
    ctx = _lib.context()
    n = 2_097_153
    t = torch.zeros(n, dtype=torch.int32, device=gpu)
    ok = torch.empty_like(t)
    ov = torch.empty_like(t)
    status = _lib.lib().bh_radix_argsort_noalloc(ctx.handle, _lib.ptr(t), _lib.ptr(t), n, 32, _lib.ptr(ok),
                                                 _lib.ptr(ov))
    assert status == 1, status
    assert "exceeds" in _lib.lib().bh_last_error(ctx.handle).decode()
