"""Input validation of the oracle: the error table of the reference's
tests/test_reference_validation.py:29-134 (ValueError / TypeError classes of
src/reference.py:57-112), restated against oracle/reference.py."""

import pytest
import torch

from oracle.reference import paged_attention_decode_reference


def _valid():
    g = torch.Generator().manual_seed(0)
    return dict(
        q=torch.randn(2, 8, 32, generator=g),
        k_cache=torch.randn(4, 16, 2, 32, generator=g),
        v_cache=torch.randn(4, 16, 2, 32, generator=g),
        block_table=torch.tensor([[0, 1], [2, 3]], dtype=torch.int32),
        seq_lens=torch.tensor([20, 20], dtype=torch.int32),
    )


def _call(**over):
    kw = _valid()
    kw.update(over)
    return paged_attention_decode_reference(**kw)


def test_valid_inputs_do_not_raise():
    _call()


def test_int64_indices_accepted():
    _call(block_table=torch.tensor([[0, 1], [2, 3]]), seq_lens=torch.tensor([20, 17]))


CASES = [
    ("q_wrong_ndim", dict(q=torch.zeros(2, 8, 32, 1)), ValueError),
    ("k_cache_wrong_ndim", dict(k_cache=torch.zeros(4, 16, 2)), ValueError),
    ("v_cache_shape_mismatch", dict(v_cache=torch.zeros(4, 16, 2, 16)), ValueError),
    ("block_table_wrong_ndim", dict(block_table=torch.zeros(2, 2, 1, dtype=torch.int32)), ValueError),
    ("seq_lens_wrong_ndim", dict(seq_lens=torch.zeros(2, 1, dtype=torch.int32)), ValueError),
    ("q_wrong_dtype", dict(q=torch.zeros(2, 8, 32, dtype=torch.float16)), TypeError),
    ("k_cache_wrong_dtype", dict(k_cache=torch.zeros(4, 16, 2, 32, dtype=torch.float16)), TypeError),
    ("v_cache_wrong_dtype", dict(v_cache=torch.zeros(4, 16, 2, 32, dtype=torch.float16)), TypeError),
    ("block_table_wrong_dtype", dict(block_table=torch.zeros(2, 2)), TypeError),
    ("seq_lens_wrong_dtype", dict(seq_lens=torch.zeros(2)), TypeError),
    ("block_table_batch_mismatch", dict(block_table=torch.zeros(3, 2, dtype=torch.int32)), ValueError),
    ("seq_lens_batch_mismatch", dict(seq_lens=torch.zeros(3, dtype=torch.int32)), ValueError),
    ("head_dim_mismatch", dict(q=torch.zeros(2, 8, 16)), ValueError),
    ("page_size_zero", dict(k_cache=torch.zeros(4, 0, 2, 32), v_cache=torch.zeros(4, 0, 2, 32)), ValueError),
    ("num_kv_heads_zero", dict(k_cache=torch.zeros(4, 16, 0, 32), v_cache=torch.zeros(4, 16, 0, 32)), ValueError),
    ("gqa_not_divisible", dict(q=torch.zeros(2, 5, 32)), ValueError),
    ("negative_seq_len", dict(seq_lens=torch.tensor([-1, 20], dtype=torch.int32)), ValueError),
    ("seq_len_exceeds_capacity", dict(seq_lens=torch.tensor([999, 20], dtype=torch.int32)), ValueError),
    ("negative_page_id", dict(block_table=torch.tensor([[-1, 1], [2, 3]], dtype=torch.int32)), ValueError),
    ("page_id_out_of_range", dict(block_table=torch.tensor([[99, 1], [2, 3]], dtype=torch.int32)), ValueError),
]


@pytest.mark.parametrize("over,exc", [pytest.param(o, e, id=i) for i, o, e in CASES])
def test_invalid_inputs_raise(over, exc):
    with pytest.raises(exc):
        _call(**over)


@pytest.mark.gpu
def test_device_mismatch_raises():
    with pytest.raises(ValueError):
        _call(k_cache=_valid()["k_cache"].cuda())
