"""Every launch of a call follows the caller's current stream: the whole call
(preprocess, k-means, quantisers, qm.K_s, attention, and the SDPA path's
dequantisation) run inside ``torch.cuda.stream(side)`` on a default-priority
side stream, while the default stream is kept busy, equals the same call on
the default stream bit for bit -- a launch on any other stream would race
with the side stream's own work."""

import pytest
import torch

from conftest import cpu_randn

pytestmark = pytest.mark.gpu

CASES = {
    "dynamic_qmk_kmeans": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                               q_kmeans_k=16, p_requant=True, p_quant="dynamic", rowmax_mode="qm_k"),
    "mx_hadamard_vsmooth_vkmeans": dict(qk_quant="mxfp8", mxfp8_block_size=32, qk_hadamard=True, v_quant="mxfp8",
                                        v_mxfp8_block_size=64, v_kmeans_k=16, v_smooth_mode="per_block",
                                        v_smooth_block_size=64, smoothing="full", q_kmeans_k=16, p_requant=True,
                                        p_quant="mx", rowmax_mode="online"),
    "blasst_mean": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                        q_kmeans_k=16, p_requant=True, p_quant="dynamic", rowmax_mode="qm_k", blasst_lambda=0.05,
                        blasst_fill="mean_a1.5"),
    "sdpa_qm": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="full", q_smooth_block_size=256,
                    q_kmeans_k=16, p_requant=False),
    "sdpa_plain": dict(qk_quant="fp8_block", fp8_block_size=64, smoothing="off", q_kmeans_k=None, p_requant=False),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_side_stream_matches_default_stream(gpu, name):
    from low_bit_fake_quant import QuantConfig, fake_quant_attention, prepare_for_attention
    cfg = QuantConfig(**CASES[name])
    q, k, v = (cpu_randn(1, 1024, 2, 128, seed=s, scale=1.5).to(gpu) for s in (1, 2, 3))
    want = fake_quant_attention(q, k, v, cfg)
    cache_want = fake_quant_attention(q, k, v, cfg, preprocess_cache=prepare_for_attention(q, k, v, cfg))
    torch.cuda.synchronize()

    side = torch.cuda.Stream(device=gpu)  # default priority
    busy = torch.randn(4096, 4096, device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    for _ in range(3):
        busy = (busy @ busy) * 1e-2  # keeps the default stream occupied while the side stream runs
        with torch.cuda.stream(side):
            got = fake_quant_attention(q, k, v, cfg)
            cache = prepare_for_attention(q, k, v, cfg)
            got_cached = fake_quant_attention(q, k, v, cfg, preprocess_cache=cache)
        side.synchronize()
        assert torch.equal(got, want), f"{name}: side-stream call differs"
        assert torch.equal(got_cached, cache_want), f"{name}: side-stream cached call differs"
    torch.cuda.synchronize()
