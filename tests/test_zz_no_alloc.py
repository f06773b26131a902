"""lbfq_kmeans_noalloc (the allocation-free k-means entry point) against
lbfq_kmeans with a caller workspace: bitwise-equal labels, order and inverse
on two calls in a row (the second on a smaller input, reusing the built-in
scratch the first call left behind), and a clear error above the limit."""

import pytest
import torch

from conftest import cpu_randn

pytestmark = pytest.mark.gpu


def _with_workspace(lib, L, x, k, iters, seed):
    b, s, h, d = x.shape
    ws = torch.empty(int(lib.lbfq_kmeans_workspace_bytes(b, s, h, d, k)), dtype=torch.uint8, device=x.device)
    out = [torch.empty((b * h, s), dtype=torch.int32, device=x.device) for _ in range(3)]
    L.check(lib.lbfq_kmeans(x.data_ptr(), L.DTYPE_CODE[x.dtype], b, s, h, d, k, iters, seed, ws.data_ptr(),
                            *(t.data_ptr() for t in out), L.stream_handle(x.device)), "lbfq_kmeans")
    return out


def _no_alloc(lib, L, x, k, iters, seed):
    b, s, h, d = x.shape
    out = [torch.empty((b * h, s), dtype=torch.int32, device=x.device) for _ in range(3)]
    L.check(lib.lbfq_kmeans_noalloc(x.data_ptr(), L.DTYPE_CODE[x.dtype], b, s, h, d, k, iters, seed,
                                    *(t.data_ptr() for t in out), L.stream_handle(x.device)), "lbfq_kmeans_noalloc")
    return out


def test_kmeans_noalloc_matches_workspace_entry(gpu):
    from low_bit_fake_quant import _lib as L
    lib = L.load()
    cases = [((1, 8192, 4, 128), 32, torch.bfloat16, 3),   # first call: the larger input
             ((1, 1000, 2, 64), 8, torch.float16, 5)]      # second call: smaller, scratch holds the first's data
    for shape, k, dtype, seed in cases:
        x = cpu_randn(*shape, seed=seed, dtype=dtype).to(gpu)
        want = _with_workspace(lib, L, x, k, 10, seed)
        got = _no_alloc(lib, L, x, k, 10, seed)
        torch.cuda.synchronize()
        for g, w, name in zip(got, want, ("labels", "order", "inverse")):
            assert torch.equal(g, w), f"{shape}: {name} differ"
        # the order is a permutation and the inverse inverts it
        ar = torch.arange(shape[1], device=gpu, dtype=torch.int32).expand(shape[0] * shape[2], -1)
        assert torch.equal(torch.gather(got[2], 1, got[1].long()), ar)


def test_kmeans_noalloc_rejects_problems_above_its_scratch(gpu):
    from low_bit_fake_quant import _lib as L
    lib = L.load()
    cap = int(lib.lbfq_kmeans_noalloc_max_workspace_bytes())
    assert cap == 64 << 20
    b, s, h, d, k = 1, 65536, 40, 128, 64                 # needs ~170 MB of workspace
    assert int(lib.lbfq_kmeans_workspace_bytes(b, s, h, d, k)) > cap
    out = torch.empty((1,), dtype=torch.int32, device=gpu)
    x = torch.empty((1,), dtype=torch.bfloat16, device=gpu)
    rc = lib.lbfq_kmeans_noalloc(x.data_ptr(), L.DTYPE_CODE[x.dtype], b, s, h, d, k, 10, 0, out.data_ptr(),
                                 out.data_ptr(), out.data_ptr(), L.stream_handle(gpu))
    assert rc == -1
    assert "built-in scratch" in lib.lbfq_last_error().decode()
