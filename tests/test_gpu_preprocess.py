"""GPU smoothing, Hadamard and k-means reorder: bit-exact vs the CPU oracle."""

import pytest
import torch

from conftest import cpu_randn
from oracle import hadamard as ohad
from oracle import kmeans as okm
from oracle import preprocess as opre

pytestmark = pytest.mark.gpu


def _k(shape, dtype, seed):
    x = cpu_randn(*shape, seed=seed, dtype=torch.float32)
    x = x + 2.0 * cpu_randn(1, 1, shape[2], shape[3], seed=seed + 1, dtype=torch.float32)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("s", [1024, 1000])
def test_smooth_k_bit_exact(gpu, dtype, s):
    from low_bit_fake_quant import smooth_k
    k = _k((2, s, 3, 128), dtype, seed=1)
    out, mean = smooth_k(k.to(gpu))
    ro, rm = opre.smooth_k(k)
    assert torch.equal(mean.cpu(), rm)
    assert torch.equal(out.cpu(), ro)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_group_mean_q_bit_exact(gpu, dtype):
    from low_bit_fake_quant import group_mean_q
    q = _k((1, 1024, 2, 64), dtype, seed=2)
    out, qm = group_mean_q(q.to(gpu), block_q=256)
    ro, rq = opre.group_mean_q(q, 256)
    assert torch.equal(qm.cpu(), rq)
    assert torch.equal(out.cpu(), ro)


def test_smooth_v_bit_exact(gpu):
    from low_bit_fake_quant import smooth_v_per_block
    v = _k((1, 512, 2, 128), torch.bfloat16, seed=3)
    out, alpha = smooth_v_per_block(v.to(gpu), block_s=64)
    ro, ra = opre.smooth_v_per_block(v, 64)
    assert torch.equal(alpha.cpu(), ra)
    assert torch.equal(out.cpu(), ro)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("random_sign", [True, False])
def test_hadamard_bit_exact(gpu, d, random_sign):
    from low_bit_fake_quant import apply_qk_hadamard, hadamard_transform_last_dim
    q = _k((1, 256, 3, d), torch.bfloat16, seed=4)
    k = _k((1, 256, 3, d), torch.bfloat16, seed=5)
    qr, kr = apply_qk_hadamard(q.to(gpu), k.to(gpu), random_sign=random_sign, seed=7)
    rq, rk = ohad.apply_qk_hadamard(q, k, random_sign=random_sign, seed=7)
    assert torch.equal(qr.cpu(), rq) and torch.equal(kr.cpu(), rk)
    x = cpu_randn(10, 7, d, seed=9, dtype=torch.float32)
    y = hadamard_transform_last_dim(x.to(gpu), scale=0.25)
    assert torch.equal(y.cpu(), ohad.fwht_last_dim(x, 0.25))


@pytest.mark.parametrize("k_clusters,iters", [(32, 10), (16, 3), (1, 2), (64, 1)])
def test_kmeans_reorder_bit_exact(gpu, k_clusters, iters):
    from low_bit_fake_quant import apply_kv_permutation, kmeans_reorder_tokens
    g = torch.Generator().manual_seed(5)
    cent = torch.randn(2, 8, 128, generator=g) * 2
    lab = torch.randint(0, 8, (1024, 2), generator=g)
    x = (torch.gather(cent.unsqueeze(0).expand(1024, 2, 8, 128), 2, lab.view(1024, 2, 1, 1).expand(1024, 2, 1, 128))
         .squeeze(2) + 0.3 * torch.randn(1024, 2, 128, generator=g)).unsqueeze(0).to(torch.bfloat16)
    r = kmeans_reorder_tokens(x.to(gpu), n_clusters=k_clusters, max_iters=iters, seed=3)
    ref = okm.kmeans_reorder_tokens(x, n_clusters=k_clusters, max_iters=iters, seed=3)
    assert torch.equal(r.labels.cpu(), ref["labels"])
    assert torch.equal(r.order.cpu(), ref["order"])
    assert torch.equal(r.inverse_order.cpu(), ref["inverse_order"])
    assert torch.equal(r.tensor_reordered.cpu(), ref["tensor_reordered"])
    y = cpu_randn(1, 1024, 2, 128, seed=8)
    assert torch.equal(apply_kv_permutation(y.to(gpu), r.order).cpu(), okm.apply_kv_permutation(y, ref["order"]))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("gathered", [False, True])
def test_qmk_table_and_rowmax(gpu, d, gathered):
    """qm . K_s table (K_s formed in-kernel from K and its column mean, through an
    optional row gather) against float64 on the CPU; rowmax is the table's row max."""
    from low_bit_fake_quant import _lib
    from low_bit_fake_quant._ops import RowSource, qmk
    s, h, g = 1000, 3, 4                      # ragged S: padding columns of the table stay zero
    k = cpu_randn(1, s, h, d, seed=21) * 3 + 1.5
    qm = cpu_randn(1, g, h, d, seed=22, dtype=torch.float32)
    mean = opre.k_mean(k)                     # (B,H,D) fp32, the smoothing mean
    gen = torch.Generator().manual_seed(23)
    order = torch.stack([torch.randperm(s, generator=gen) for _ in range(h)]).to(torch.int32) if gathered else None
    src = RowSource(k.to(gpu), gather=order.to(gpu) if gathered else None, sub_mode=_lib.SUB_COLVEC,
                    sub=mean.to(gpu))
    scale = 0.127
    pitch = 1024
    bias, rowmax = qmk(qm.to(gpu), src, scale, s_pitch=pitch)
    bias, rowmax = bias.cpu(), rowmax.cpu()
    kk = k.permute(0, 2, 1, 3)                                         # (B,H,S,D)
    if gathered:
        kk = torch.stack([kk[0, i, order[i].long()] for i in range(h)]).unsqueeze(0)
    ks = (kk.float() - mean[:, :, None, :]).to(torch.bfloat16).double()   # the quantiser's rounding
    ref = torch.einsum("bghd,bhnd->bhgn", qm.double(), ks) * scale
    mag = torch.einsum("bghd,bhnd->bhgn", qm.double().abs(), ks.abs()) * scale
    got = bias[..., :s].double()
    assert ((got - ref).abs() <= 1e-6 * mag + 1e-30).all()
    assert torch.count_nonzero(bias[..., s:]) == 0
    assert torch.equal(rowmax, bias[..., :s].amax(-1))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("blk", [16, 32, 64])
@pytest.mark.parametrize("gathered", [False, True])
def test_qmk_fused_k_quant_matches_separate_passes(gpu, d, blk, gathered):
    """lbfq_qmk_kquant: the qm.K_s table, row maxima, K_s codes and block scales
    equal (bitwise) those of lbfq_qmk plus the row-tile fp8_block quantiser, and
    the codes / scales equal the CPU oracle's fp8_block quant of K_s.  S = 960
    leaves a partial last workgroup (256 keys each)."""
    from oracle import quant as oq
    from low_bit_fake_quant import _lib
    from low_bit_fake_quant._ops import RowSource, qmk, rowtile
    s, h, g, pitch = 960, 3, 4, 1024
    k = (cpu_randn(1, s, h, d, seed=31) * 3 + 1.5).to(torch.bfloat16)
    qm = cpu_randn(1, g, h, d, seed=32, dtype=torch.float32)
    mean = opre.k_mean(k)
    gen = torch.Generator().manual_seed(33)
    order = torch.stack([torch.randperm(s, generator=gen) for _ in range(h)]).to(torch.int32) if gathered else None
    src = RowSource(k.to(gpu), gather=order.to(gpu) if gathered else None, sub_mode=_lib.SUB_COLVEC,
                    sub=mean.to(gpu))
    nb = s // blk
    codes_a = torch.zeros((1, h, pitch, d), dtype=torch.uint8, device=gpu)
    scale_a = torch.empty((1, h, nb), dtype=torch.float32, device=gpu)
    rowtile(src, R=blk, quant_mode=_lib.Q_FP8_BLOCK, codes=codes_a, codes_layout=_lib.LAYOUT_BHSD,
            codes_spitch=pitch, scale=scale_a, scale_strides=(h * nb, 1, nb, 0))
    bias_a, rowmax_a = qmk(qm.to(gpu), src, 0.127, s_pitch=pitch)
    codes_b = torch.zeros((1, h, pitch, d), dtype=torch.uint8, device=gpu)
    scale_b = torch.full((1, h, nb), -1.0, dtype=torch.float32, device=gpu)
    bias_b, rowmax_b = qmk(qm.to(gpu), src, 0.127, s_pitch=pitch, k_quant=(codes_b, scale_b, blk))
    assert torch.equal(codes_b, codes_a) and torch.equal(scale_b, scale_a)
    assert torch.equal(bias_b, bias_a) and torch.equal(rowmax_b, rowmax_a)
    # the oracle's fp8_block quant of K_s (NHD, gathered rows in output order)
    kk = k.permute(0, 2, 1, 3)
    if gathered:
        kk = torch.stack([kk[0, i, order[i].long()] for i in range(h)]).unsqueeze(0)
    ks = (kk.float() - mean[:, :, None, :]).to(torch.bfloat16).permute(0, 2, 1, 3)   # (B,S,H,D)
    oc, osc = oq.fp8_block_quant(ks, block_s=blk)
    assert torch.equal(codes_b.cpu()[:, :, :s], oc.permute(0, 2, 1, 3))
    assert torch.equal(scale_b.cpu(), osc.permute(0, 2, 1))


@pytest.mark.parametrize("iters", [10, 14])
def test_kmeans_converged_slices_skip_later_rounds_bit_exact(gpu, iters):
    """A slice whose assignment leaves every label unchanged has converged and
    skips its later rounds; the result equals the oracle, which runs every
    round.  Head 0 holds 32 well-separated clusters, one per initial stride
    block (converged after two rounds: the skip path), head 1 pure noise
    (labels still changing in the last round: no skip), in the same call."""
    from low_bit_fake_quant import kmeans_reorder_tokens
    g = torch.Generator().manual_seed(11)
    cent = torch.randn(32, 128, generator=g) * 8
    x0 = cent[torch.arange(2048) // 64] + 0.05 * torch.randn(2048, 128, generator=g)
    x1 = torch.randn(2048, 128, generator=g)
    x = torch.stack([x0, x1], 1).unsqueeze(0).to(torch.bfloat16)   # (1, S, H=2, D)

    def labels_after(r):
        return okm.kmeans_reorder_tokens(x, n_clusters=32, max_iters=r, seed=7)["labels"]
    conv = [next((r for r in range(1, iters) if torch.equal(labels_after(r)[hh], labels_after(r + 1)[hh])), None)
            for hh in (0, 1)]
    assert conv[0] is not None and conv[0] < iters - 1, f"head 0 should converge early: {conv}"
    assert conv[1] is None, f"head 1 should still change in the last round: {conv}"
    r = kmeans_reorder_tokens(x.to(gpu), n_clusters=32, max_iters=iters, seed=7)
    ref = okm.kmeans_reorder_tokens(x, n_clusters=32, max_iters=iters, seed=7)
    assert torch.equal(r.labels.cpu(), ref["labels"])
    assert torch.equal(r.order.cpu(), ref["order"])
    assert torch.equal(r.tensor_reordered.cpu(), ref["tensor_reordered"])
