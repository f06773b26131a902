"""A whole fake_quant_attention call can be captured in a HIP graph
(``torch.cuda.graph``) and replayed: the call makes no host synchronisation
and no memset (buffers are cleared by fill kernels), and every launch follows
the capturing stream.  Each replay -- with eager work and new input values
copied into the captured inputs between replays -- equals an eager call on
the same inputs bit for bit."""

import pytest
import torch

from conftest import cpu_randn

pytestmark = pytest.mark.gpu

CASES = {
    "dynamic_qmk_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                               q_kmeans_k=16, p_requant=True, p_quant="dynamic", rowmax_mode="qm_k"),
    "blasst_mean": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                        q_kmeans_k=16, p_requant=True, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05,
                        blasst_fill="mean_a1.5"),
    "mx_hadamard_vsmooth_vkmeans": dict(qk_quant="mxfp8", mxfp8_block_size=32, qk_hadamard=True, v_quant="mxfp8",
                                        v_mxfp8_block_size=64, v_kmeans_k=16, v_smooth_mode="per_block",
                                        v_smooth_block_size=64, smoothing="full", q_kmeans_k=16, p_requant=True,
                                        p_quant="mx", rowmax_mode="online"),
    "sdpa_plain": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="off", q_kmeans_k=None, p_requant=False),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_graph_replays_match_eager_calls(gpu, name):
    from low_bit_fake_quant import QuantConfig, fake_quant_attention
    cfg = QuantConfig(**CASES[name])
    shape = (1, 1024, 2, 128)
    q, k, v = (cpu_randn(*shape, seed=s, scale=1.5).to(gpu) for s in (1, 2, 3))

    side = torch.cuda.Stream(device=gpu)  # default priority
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):  # warm-up (first-call set-up) outside the capture
        for _ in range(2):
            fake_quant_attention(q, k, v, cfg)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fake_quant_attention(q, k, v, cfg)
    torch.cuda.synchronize()

    for rep in range(4):
        if rep >= 2:  # new values in the captured inputs
            for t, s in zip((q, k, v), (10 * rep + 1, 10 * rep + 2, 10 * rep + 3)):
                t.copy_(cpu_randn(*shape, seed=s, scale=1.5).to(gpu))
        g.replay()
        eager_other = fake_quant_attention(v, q, k, cfg)  # eager work between replays
        torch.cuda.synchronize()
        want = fake_quant_attention(q, k, v, cfg)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"{name}: replay {rep} differs from the eager call"
        assert torch.isfinite(eager_other.float()).all()
