"""GPU parity of the DSA top-k page-table transform (fagq_dsa_topk_launch)
against the CPU oracle (oracle/dsa_topk_oracle.c): integer outputs, so the
bar is bit-exact equality of out_blocks and out_pages."""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import note

pytestmark = pytest.mark.gpu


def run_both(pkg, dev, scores, page_table, q_pos, kv_lens, bs, k):
    B, H, Q, NB = scores.shape
    ob = torch.full((B, H, Q, k), -7, dtype=torch.int32, device=dev)
    op = torch.full((B, H, Q, k), -7, dtype=torch.int32, device=dev)
    pkg.dsa_topk_page_table_transform(scores.to(dev), page_table.to(dev), q_pos.to(dev),
                                      kv_lens.to(dev), ob, op, bs, k)
    torch.cuda.synchronize()
    s_np = scores.view(torch.uint16).numpy() if scores.dtype == torch.bfloat16 else scores.numpy()
    rb, rp = oracle.dsa_topk(s_np, page_table.numpy(), q_pos.numpy(), kv_lens.numpy(), bs, k)
    return ob.cpu().numpy(), op.cpu().numpy(), rb, rp


def check(pkg, dev, scores, page_table, q_pos, kv_lens, bs, k, label):
    note(f"dsa {label}: shape {tuple(scores.shape)} {scores.dtype} k={k} bs={bs}")
    gb, gp, rb, rp = run_both(pkg, dev, scores, page_table, q_pos, kv_lens, bs, k)
    bad = np.argwhere((gb != rb).any(-1))
    assert bad.size == 0, f"{label}: {len(bad)} rows differ, first {bad[0].tolist()}: " \
                          f"gpu {gb[tuple(bad[0])][:8]} ref {rb[tuple(bad[0])][:8]}"
    assert np.array_equal(gp, rp), label


def case(seed, B=2, H=2, Q=24, NB=512, bs=16, dtype=torch.float32, ties=None, idx=torch.int32):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B, H, Q, NB, generator=g)
    if ties == "round":
        s = torch.round(s * 2) / 2
    elif ties == "heavy":
        s = torch.where(torch.rand(s.shape, generator=g) < 0.8, torch.ones_like(s), s)
    elif ties == "equal":
        s = torch.full_like(s, 0.25)
    elif ties == "outlier":                  # one huge score stretches the fp32 range
        s[..., 3] = 1e30
    elif ties == "cluster":                  # half the row in a narrow band above the rest
        s = torch.where(torch.rand(s.shape, generator=g) < 0.5, 5 + 1e-4 * s, s)
    elif ties == "offset":                   # range tiny next to the magnitude: degenerate bin map
        s = 1000 + 1e-3 * s
    elif ties == "offset_lin":               # large bin offset (|vmin s| ~ 4e4), still linear
        s = 10 + 1e-2 * s
    s[torch.rand(s.shape, generator=g) < 0.01] = float("-inf")
    s = s.to(dtype)
    kv = torch.randint(0, NB * bs + 2 * bs, (B,), generator=g).to(idx)
    pos = torch.randint(-3, NB * bs, (B, Q), generator=g).to(idx)
    pos[:, 0] = NB * bs - 1                  # a full-length row in every batch
    pt = torch.randint(0, 1 << 24, (B, NB), generator=g).to(torch.int32)
    return s, pt, pos, kv


@pytest.mark.parametrize("NB", [64, 512, 1000, 2048, 4096])
@pytest.mark.parametrize("k", [1, 32, 128])
def test_dsa_random(pkg, gpu, NB, k):
    s, pt, pos, kv = case(NB + k, NB=NB)
    check(pkg, gpu, s, pt, pos, kv, 16, k, f"random NB={NB}")


@pytest.mark.parametrize("ties", ["round", "heavy", "equal", "outlier", "cluster", "offset",
                                  "offset_lin"])
@pytest.mark.parametrize("NB,k", [(4096, 128), (2048, 64), (1024, 256)])
def test_dsa_ties(pkg, gpu, ties, NB, k):
    s, pt, pos, kv = case(7, NB=NB, ties=ties)
    check(pkg, gpu, s, pt, pos, kv, 8, k, f"ties={ties}")


@pytest.mark.parametrize("dtype,idx", [(torch.bfloat16, torch.int32), (torch.float32, torch.int64),
                                       (torch.bfloat16, torch.int64)])
def test_dsa_dtypes(pkg, gpu, dtype, idx):
    s, pt, pos, kv = case(3, NB=4096, dtype=dtype, idx=idx)
    check(pkg, gpu, s, pt, pos, kv, 64, 128, f"{dtype} {idx}")


def test_dsa_special_values(pkg, gpu):
    s, pt, pos, kv = case(11, NB=512, Q=8)
    s[0, 0, 0, 5] = float("inf")
    s[0, 0, 1, :] = float("-inf")
    s[0, 1, 2, ::2] = -0.0
    s[0, 1, 2, 1::2] = 0.0
    s[1, 0, 3, :300] = 1e-42                 # subnormals
    s[1, 1, 4, :] = torch.linspace(-1e38, 1e38, 512)
    pos[1, 5] = -1
    kv[0] = max(int(kv[0]), 512 * 16)
    check(pkg, gpu, s, pt, pos, kv, 16, 64, "special values")


@pytest.mark.parametrize("bs", [1, 3, 100])
def test_dsa_odd_block_sizes(pkg, gpu, bs):
    s, pt, pos, kv = case(21 + bs, NB=1000, bs=bs)
    check(pkg, gpu, s, pt, pos, kv, bs, 64, f"block_size={bs}")


def test_dsa_int64_positions_past_2_31(pkg, gpu):
    s, pt, pos, kv = case(31, NB=1024, Q=16, idx=torch.int64)
    g = torch.Generator().manual_seed(5)
    bs = 1 << 22
    kv[0], kv[1] = 1 << 33, (1 << 31) + 5 * bs
    pos[0] = torch.randint(-2, 1 << 34, (16,), generator=g)
    pos[1] = torch.randint(0, 1 << 32, (16,), generator=g)
    pos[1, 0] = (1 << 31) + 5 * bs - 1
    check(pkg, gpu, s, pt, pos, kv, bs, 128, "int64 positions past 2^31")


def test_dsa_zero_kv_and_negative_pos(pkg, gpu):
    s, pt, pos, kv = case(12, NB=512, Q=8)
    kv[1] = 0
    pos[0, :4] = -1
    check(pkg, gpu, s, pt, pos, kv, 16, 32, "empty rows")


@pytest.mark.parametrize("name", ["dsa_f32_b2h32q512_nb4096_k128_bs64",
                                  "dsa_f32_b1h32q1024_nb2048_k64_bs64",
                                  "dsa_f32_b2h16q256_nb1024_k64_bs128",
                                  "dsa_bf16_b2h32q512_nb4096_k128_bs64"])
def test_dsa_reference_workloads_full_size(pkg, gpu, name):
    from fagq_mi355x.workloads import DSA_CONFIGS, make_dsa_inputs
    w = DSA_CONFIGS[name]
    s, pt, pos, kv = make_dsa_inputs(w)
    check(pkg, gpu, s, pt, pos, kv, w.block_size, w.top_k, name)


def test_dsa_python_errors(pkg, gpu):
    s = torch.zeros(1, 1, 2, 64, device=gpu)
    pt = torch.zeros(1, 64, dtype=torch.int32, device=gpu)
    pos = torch.zeros(1, 2, dtype=torch.int32, device=gpu)
    kv = torch.zeros(1, dtype=torch.int32, device=gpu)
    ob = torch.empty(1, 1, 2, 8, dtype=torch.int32, device=gpu)
    op = torch.empty_like(ob)
    with pytest.raises(TypeError):
        pkg.dsa_topk_page_table_transform(s.half(), pt, pos, kv, ob, op, 16, 8)
    with pytest.raises(TypeError):
        pkg.dsa_topk_page_table_transform(s, pt, pos.long(), kv, ob, op, 16, 8)
    with pytest.raises(ValueError):
        pkg.dsa_topk_page_table_transform(s, pt, pos, kv, ob[..., :4], op, 16, 8)
    with pytest.raises(pkg.FagqError):
        pkg.dsa_topk_page_table_transform(s, pt, pos, kv, ob, op, 0, 8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("NB,k", [(4095, 128), (6000, 64), (8192, 128), (16384, 256), (1021, 32)])
def test_dsa_any_row_length(pkg, gpu, dtype, NB, k):
    """Row lengths that are not a multiple of the 16-byte vector (per-score
    loads) and rows of up to 16 chunks of 1024 blocks (16 waves)."""
    s, pt, pos, kv = case(NB + k, B=2, H=2, Q=12, NB=NB, dtype=dtype)
    check(pkg, gpu, s, pt, pos, kv, 16, k, f"NB={NB} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("NB,ties", [(40000, None), (40001, "heavy"), (70000, "round"),
                                     (20480, "outlier")])
def test_dsa_rows_longer_than_16_chunks(pkg, gpu, dtype, NB, ties):
    """More than 16 chunks: each wave walks several chunks and reads the row
    again in every pass (also through the radix refinement with ties)."""
    s, pt, pos, kv = case(NB, B=1, H=2, Q=6, NB=NB, dtype=dtype, ties=ties)
    check(pkg, gpu, s, pt, pos, kv, 8, 128, f"NB={NB} ties={ties} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("offset", [1, 2, 3])
def test_dsa_scores_not_16_byte_aligned(pkg, gpu, dtype, offset):
    """A scores tensor that starts 1..3 elements into its allocation: rows are
    read one score per load, with the same result."""
    s, pt, pos, kv = case(50 + offset, B=2, H=2, Q=10, NB=2048, dtype=dtype)
    flat = torch.empty(s.numel() + offset, dtype=dtype)
    flat[offset:] = s.reshape(-1)
    note(f"dsa unaligned offset={offset} {dtype}")
    B, H, Q, NB = s.shape
    sd = torch.empty(s.numel() + offset, dtype=dtype, device=gpu)[offset:].view(B, H, Q, NB)
    sd.copy_(s.to(gpu))
    assert sd.data_ptr() % 16 != 0
    ob = torch.full((B, H, Q, 64), -7, dtype=torch.int32, device=gpu)
    op = torch.full((B, H, Q, 64), -7, dtype=torch.int32, device=gpu)
    pkg.dsa_topk_page_table_transform(sd, pt.to(gpu), pos.to(gpu), kv.to(gpu), ob, op, 16, 64)
    torch.cuda.synchronize()
    s_np = s.view(torch.uint16).numpy() if dtype == torch.bfloat16 else s.numpy()
    rb, rp = oracle.dsa_topk(s_np, pt.numpy(), pos.numpy(), kv.numpy(), 16, 64)
    assert np.array_equal(ob.cpu().numpy(), rb) and np.array_equal(op.cpu().numpy(), rp)


# top_k past 256 (the reference's power-of-two top_k up to its 1024-block chunk width,
# task02.py:913-945 and :1712-1725) takes the kernel with the larger candidate array;
# 257 is the first such top_k, 256 the last of the smaller one.
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("NB,k", [(1024, 512), (1024, 1024), (4096, 512), (4096, 1024),
                                  (8192, 512), (8192, 1024), (4096, 256), (4096, 257),
                                  (2000, 1000)])
def test_dsa_large_top_k(pkg, gpu, dtype, NB, k):
    s, pt, pos, kv = case(NB + k, B=2, H=2, Q=16, NB=NB, bs=16, dtype=dtype)
    check(pkg, gpu, s, pt, pos, kv, 16, k, f"large_k NB={NB} k={k}")


@pytest.mark.parametrize("ties", ["round", "heavy", "equal", "outlier", "cluster"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("NB,k", [(4096, 1024), (8192, 512)])
def test_dsa_large_top_k_ties(pkg, gpu, ties, dtype, NB, k):
    s, pt, pos, kv = case(7 * NB + k, B=1, H=2, Q=12, NB=NB, bs=16, dtype=dtype, ties=ties)
    check(pkg, gpu, s, pt, pos, kv, 16, k, f"large_k ties={ties} NB={NB} k={k}")


def test_dsa_large_top_k_all_rows_valid(pkg, gpu):
    # Every row sees the whole NB-block prefix: exactly top_k of NB selected.
    g = torch.Generator().manual_seed(11)
    B, H, Q, NB, bs, k = 1, 4, 32, 4096, 64, 1024
    s = torch.randn(B, H, Q, NB, generator=g)
    pt = torch.randint(0, 1 << 24, (B, NB), generator=g).to(torch.int32)
    pos = torch.full((B, Q), NB * bs - 1, dtype=torch.int32)
    kv = torch.full((B,), NB * bs, dtype=torch.int32)
    check(pkg, gpu, s, pt, pos, kv, bs, k, "large_k all rows valid")
