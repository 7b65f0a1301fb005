"""The reference's own grouped-decode GPU tests at their exact shapes, against the float64
oracle (tests/test_native_draft_decode_gpu.py:63-135 in the reference): 12 query heads,
2 kv heads, head dim 256, 16-token pages handed to each row in reverse logical order (so
that a page-table mistake cannot pass by accident), the page table built from flat
``kv_indptr`` / ``kv_indices`` lists, fp16 and e5m2 pools, lengths [37, 53], [67] and
[41, 67]. The reference checks against SDPA at 2e-2; the bound here is the oracle's
2e-3 + half an output ulp. The dense e5m2 decode case of
tests/test_qsa_kernels_gpu.py:233-303 (6 query heads on 1 kv head, lengths [200, 480],
seeds 40 and 50) runs here too. The reference's extend GPU test shape runs in
tests/test_gpu_extend.py (test_extend_reference_gpu_test_shape).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from tests.helpers import assert_attn_close, to_f64

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _row_tokens(pages, page_size, length):
    return [p * page_size + i for p in pages for i in range(page_size)][:length]


@pytest.mark.parametrize("lengths,dtype", [
    ([37, 53], torch.float16),
    ([67], torch.float16),
    ([41, 67], torch.float8_e5m2),
])
def test_grouped_decode_reference_gpu_test_shape(lengths, dtype):
    from sglang_restomod_amd.attention.mi355x import draft_decode_plan as plan
    from sglang_restomod_amd.attention.mi355x import ops

    heads, heads_kv, dim, page_size = 12, 2, 256, 16
    print(f"[case] lengths={lengths} dtype={dtype}", flush=True)
    gen = torch.Generator().manual_seed(0)
    pages_per_row = [(n + page_size - 1) // page_size for n in lengths]
    total_pages = sum(pages_per_row)
    k_cache = torch.randn(total_pages, page_size, heads_kv, dim, generator=gen).to(torch.float16).to(dtype)
    v_cache = k_cache.clone()
    q = torch.randn(len(lengths), heads, dim, generator=gen).to(torch.float16)
    index_rows, nxt = [], 0
    for n, cnt in zip(lengths, pages_per_row):
        index_rows.append(_row_tokens(list(range(nxt, nxt + cnt))[::-1], page_size, n))
        nxt += cnt
    kv_indices = torch.tensor([t for row in index_rows for t in row], dtype=torch.int64, device=DEV)
    kv_indptr = torch.zeros(len(lengths) + 1, dtype=torch.int32, device=DEV)
    kv_indptr[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int32, device=DEV), 0)
    page_table = torch.zeros(len(lengths), max(pages_per_row), dtype=torch.int32, device=DEV)
    seq_lens = torch.zeros(len(lengths), dtype=torch.int32, device=DEV)
    rows = plan.page_table_from_indices(kv_indptr, kv_indices, page_table, seq_lens, page_size)
    assert rows == len(lengths) and seq_lens.tolist() == lengths

    scale = 1.0 / math.sqrt(dim)
    out = ops.grouped_decode_forward(q.to(DEV), k_cache.to(DEV), v_cache.to(DEV), page_table, seq_lens,
                                     softmax_scale=scale)
    torch.cuda.synchronize()

    flat_k = k_cache.float().reshape(-1, heads_kv, dim).numpy().astype(np.float64)
    flat_v = v_cache.float().reshape(-1, heads_kv, dim).numpy().astype(np.float64)
    slots = [np.asarray(row, dtype=np.int64) for row in index_rows]
    ref = oracle.paged_attention(to_f64(q), flat_k, flat_v, slots, list(range(len(lengths) + 1)),
                                 [n - 1 for n in lengths], lengths, softmax_scale=scale, causal=True)
    assert_attn_close(out, ref, what=f"grouped decode {lengths} {dtype}")


@pytest.mark.parametrize("seed", [40, 50])
def test_grouped_decode_dense_e5m2_shape(seed):
    """The reference's dense e5m2 decode case (tests/test_qsa_kernels_gpu.py:233-303):
    head dim 256, 6 query heads on 1 kv head, e5m2 K and V, 16-token pages, every row's
    page table a random permutation of the same 32 pages, lengths [200, 480], fp16
    queries. The reference bound is 3e-3; here the oracle's."""
    from sglang_restomod_amd.attention.mi355x import ops

    dim, page_size, pages, lengths = 256, 16, 32, [200, 480]
    print(f"[case] dense e5m2 seed={seed}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    k_cache = torch.randn(pages, page_size, 1, dim, generator=gen).to(torch.float8_e5m2)
    v_cache = torch.randn(pages, page_size, 1, dim, generator=gen).to(torch.float8_e5m2)
    page_table = torch.stack([torch.randperm(pages, generator=gen) for _ in lengths]).to(torch.int32)
    q = torch.randn(len(lengths), 6, dim, generator=gen).to(torch.float16)
    scale = dim ** -0.5
    out = ops.grouped_decode_forward(q.to(DEV), k_cache.to(DEV), v_cache.to(DEV), page_table.to(DEV),
                                     torch.tensor(lengths, dtype=torch.int32, device=DEV), softmax_scale=scale)
    torch.cuda.synchronize()

    flat_k = k_cache.float().reshape(-1, 1, dim).numpy().astype(np.float64)
    flat_v = v_cache.float().reshape(-1, 1, dim).numpy().astype(np.float64)
    offs = np.arange(page_size)
    slots = [(page_table[r, : (n + page_size - 1) // page_size].numpy().astype(np.int64)[:, None] * page_size
              + offs[None, :]).reshape(-1)[:n] for r, n in enumerate(lengths)]
    ref = oracle.paged_attention(to_f64(q), flat_k, flat_v, slots, list(range(len(lengths) + 1)),
                                 [n - 1 for n in lengths], lengths, softmax_scale=scale, causal=True)
    assert_attn_close(out, ref, what=f"dense e5m2 decode seed {seed}")
