"""CSR page-index conversions on the CPU - test infrastructure only.

* ``paged_kv_indices`` restates ``_paged_kv_indices`` of the reference's
  FlashInfer adapter (src/flashinfer_adapter.py:40-65), as a plain Python
  loop over the batch: sequence i uses ``ceil(seq_lens[i] / page_size)``
  pages; ``indices`` concatenates ``block_table[i, :pages_i]``; ``indptr``
  is the running page count; ``last_page_len_i = seq_lens[i] - (pages_i -
  1) * page_size`` (so a sequence with no pages gets ``page_size``, as the
  reference's formula gives).
* ``csr_to_dense`` is its inverse for the oracle: it rebuilds ``seq_lens``
  and a dense ``block_table`` (unused columns filled with ``fill``) from a
  CSR triple, so CSR inputs can be checked with ``reference.
  paged_attention_decode_reference``.

Pinned by ``tests/test_csr.py``: hand-computed known answers (page-boundary
remainder / exact-multiple / empty cases), the dense -> CSR -> dense round
trip on seeded ragged batches, and ``seq_len == (pages - 1) * page_size +
last_page_len`` for every non-empty sequence.
"""

from __future__ import annotations

import torch


def paged_kv_indices(block_table: torch.Tensor, seq_lens: torch.Tensor, page_size: int):
    """(indptr int32 [B+1], indices int32 [sum pages], last_page_len int32 [B])."""
    batch = block_table.shape[0]
    indptr = [0]
    indices = []
    last = []
    for i in range(batch):
        n = int(seq_lens[i])
        pages = -(-n // page_size)
        indices.extend(int(x) for x in block_table[i, :pages])
        indptr.append(indptr[-1] + pages)
        last.append(n - (pages - 1) * page_size)
    return (torch.tensor(indptr, dtype=torch.int32), torch.tensor(indices, dtype=torch.int32),
            torch.tensor(last, dtype=torch.int32))


def csr_to_dense(indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor, page_size: int,
                 fill: int = 0):
    """(block_table int32 [B, max pages], seq_lens int32 [B]) equivalent to a CSR triple."""
    batch = last_page_len.shape[0]
    pages = [int(indptr[i + 1]) - int(indptr[i]) for i in range(batch)]
    width = max(max(pages, default=0), 1)
    bt = torch.full((batch, width), fill, dtype=torch.int32)
    lens = []
    for i in range(batch):
        start = int(indptr[i])
        for j in range(pages[i]):
            bt[i, j] = int(indices[start + j])
        lens.append((pages[i] - 1) * page_size + int(last_page_len[i]) if pages[i] > 0 else 0)
    return bt, torch.tensor(lens, dtype=torch.int32)
