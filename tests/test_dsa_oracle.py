"""Pins the CPU oracle of the Task 02 DSA top-k page-table transform
(oracle/dsa_topk_oracle.c) before it checks the GPU.

The reference repository holds no tests or golden vectors for Task 02.  The
oracle is pinned by:
* an independent restatement: the validity rule of
  src/task02_dsa_topk_page_table_transform.py:160-167 written as vectorized
  numpy, and the order (score descending, block id ascending) as np.lexsort;
* known answers for every case the reference's masks define: negative
  q_pos, kv_len 0, a causal prefix shorter than top_k, -inf scores, ties
  (including -0 == +0), kv_len past NB blocks, and bf16 scores.
"""
import numpy as np
import pytest
import torch

import oracle


def numpy_ref(scores, page_table, q_pos, kv_lens, bs, k):
    scores = scores if scores.dtype == np.float32 else \
        (scores.astype(np.uint32) << 16).view(np.float32)
    B, H, Q, NB = scores.shape
    ob = np.full((B, H, Q, k), -1, np.int32)
    op = np.full((B, H, Q, k), -1, np.int32)
    ids = np.arange(NB)
    for b in range(B):
        valid_blocks = min(-(-int(kv_lens[b]) // bs), NB)
        for q in range(Q):
            pos = int(q_pos[b, q])
            last = min(pos // bs if pos >= 0 else -1, valid_blocks - 1)
            valid = (pos >= 0) & (ids <= last)
            for h in range(H):
                v = scores[b, h, q]
                sel = valid & (v != -np.inf)
                cand = ids[sel]
                order = np.lexsort((cand, -v[sel]))[:k]
                top = cand[order]
                ob[b, h, q, :len(top)] = top
                op[b, h, q, :len(top)] = page_table[b, top]
    return ob, op


def rand_case(seed, B=2, H=3, Q=40, NB=300, bs=16, bf16=False, ties=False):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((B, H, Q, NB)).astype(np.float32)
    if ties:
        s = np.round(s * 2) / 2                     # many exact ties
        s[s == 0] = np.where(rng.random((s == 0).sum()) < 0.5, -0.0, 0.0)
    s[rng.random(s.shape) < 0.02] = -np.inf
    if bf16:
        s = oracle.bf16_from_f32(s)
    kv = rng.integers(0, NB * bs + 3 * bs, size=B).astype(np.int32)
    pos = rng.integers(-5, NB * bs, size=(B, Q)).astype(np.int32)
    pt = rng.integers(0, 1 << 20, size=(B, NB)).astype(np.int32)
    return s, pt, pos, kv


@pytest.mark.parametrize("seed,kw", [(0, {}), (1, dict(ties=True)), (2, dict(bf16=True)),
                                     (3, dict(NB=64, bs=1)), (4, dict(NB=1024, Q=8, bs=64)),
                                     (5, dict(ties=True, bf16=True))])
@pytest.mark.parametrize("k", [1, 16, 64])
def test_oracle_matches_numpy_restatement(seed, kw, k):
    s, pt, pos, kv = rand_case(seed, **kw)
    bs = kw.get("bs", 16)
    got = oracle.dsa_topk(s, pt, pos, kv, bs, k)
    want = numpy_ref(s, pt, pos, kv, bs, k)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def one_row(v, pos=10 ** 6, kv=10 ** 6, bs=1, k=4):
    NB = len(v)
    s = np.asarray(v, np.float32).reshape(1, 1, 1, NB)
    pt = (1000 + np.arange(NB)).astype(np.int32).reshape(1, NB)
    return oracle.dsa_topk(s, pt, np.array([[pos]], np.int32), np.array([kv], np.int32), bs, k)


def test_known_answers():
    # descending order, ties by id, pages gathered
    b, p = one_row([0.5, 2.0, 2.0, -1.0, 3.0])
    assert b.ravel().tolist() == [4, 1, 2, 0] and p.ravel().tolist() == [1004, 1001, 1002, 1000]
    # -0 == +0: tie broken by id
    b, _ = one_row([-0.0, 0.0, -0.0, 0.0], k=4)
    assert b.ravel().tolist() == [0, 1, 2, 3]
    # -inf is never selected; short rows pad with -1
    b, p = one_row([-np.inf, 1.0, -np.inf, 0.0], k=4)
    assert b.ravel().tolist() == [1, 3, -1, -1] and p.ravel().tolist() == [1001, 1003, -1, -1]
    # +inf is selectable and first
    b, _ = one_row([1.0, np.inf, 2.0], k=2)
    assert b.ravel().tolist() == [1, 2]
    # negative position: nothing valid
    b, p = one_row([1.0, 2.0], pos=-1, k=2)
    assert b.ravel().tolist() == [-1, -1] and p.ravel().tolist() == [-1, -1]
    # kv_len 0: nothing valid
    b, _ = one_row([1.0, 2.0], kv=0, k=2)
    assert b.ravel().tolist() == [-1, -1]
    # causal prefix: pos 5 with block_size 4 -> blocks 0 and 1
    b, _ = one_row([0.0, 1.0, 9.0, 9.0], pos=5, bs=4, k=3)
    assert b.ravel().tolist() == [1, 0, -1]
    # kv_len limits: 9 tokens, block 4 -> 3 blocks (ceil), even for a later position
    b, _ = one_row([0.0, 1.0, 2.0, 9.0], pos=100, kv=9, bs=4, k=4)
    assert b.ravel().tolist() == [2, 1, 0, -1]
    # kv_len past NB blocks: clipped to NB
    b, _ = one_row([3.0, 1.0, 2.0], pos=10 ** 6, kv=10 ** 6, bs=4, k=4)
    assert b.ravel().tolist() == [0, 2, 1, -1]


def test_all_equal_scores_take_lowest_ids():
    b, _ = one_row([7.0] * 50, k=8)
    assert b.ravel().tolist() == list(range(8))


def test_int64_indices_and_bf16_agree_with_fp32():
    s, pt, pos, kv = rand_case(9, NB=200)
    a = oracle.dsa_topk(s, pt, pos, kv, 16, 32)
    c = oracle.dsa_topk(s, pt, pos.astype(np.int64), kv.astype(np.int64), 16, 32)
    assert np.array_equal(a[0], c[0]) and np.array_equal(a[1], c[1])
    sb = oracle.bf16_from_f32(s)
    wide = (sb.astype(np.uint32) << 16).view(np.float32)
    d = oracle.dsa_topk(sb, pt, pos, kv, 16, 32)
    e = oracle.dsa_topk(wide, pt, pos, kv, 16, 32)
    assert np.array_equal(d[0], e[0]) and np.array_equal(d[1], e[1])
    t = torch.from_numpy(s).bfloat16().view(torch.uint16).numpy()
    assert np.array_equal(t, sb)        # the bf16 bits are torch's RNE cast
