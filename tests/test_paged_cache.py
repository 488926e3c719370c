"""Block allocator and block tables of the paged decode cache (host logic only)."""
import numpy as np
import pytest

from rngd_pd_amd.engines.paged_cache import BlockAllocator, PagedKVCache


def test_allocator_exhaustion_and_reuse():
    a = BlockAllocator(10)
    x = a.allocate(4)
    y = a.allocate(6)
    assert sorted(x + y) == list(range(10)) and a.free_blocks() == 0
    with pytest.raises(MemoryError):
        a.allocate(1)
    a.release(x)
    assert sorted(a.allocate(4)) == sorted(x)


def test_seeded_allocator_is_a_permutation():
    a = BlockAllocator(64, seed=3)
    got = a.allocate(64)
    assert sorted(got) == list(range(64)) and got != list(range(64))


def test_tables_and_growth():
    c = PagedKVCache(n_layers=2, num_blocks=12, n_kv_heads=2, head_dim=64, device="cpu")
    t = c.allocate("a", 33)                       # 3 blocks
    assert t.dtype.is_floating_point is False and t.numel() == 3
    c.ensure("a", 49)                             # 4 blocks
    assert len(c.blocks("a")) == 4
    c.allocate("b", 16)
    tb = c.batch_tables(["a", "b"]).numpy()
    assert tb.shape == (2, 4) and (tb[1, 1:] == -1).all()
    assert set(tb[0]) | {tb[1, 0]} == set(c.blocks("a")) | set(c.blocks("b"))
    with pytest.raises(KeyError):
        c.allocate("a", 1)
    c.free("a")
    assert c.alloc.free_blocks() == 12 - 1
    v = c.view("z", 20, S=64)
    assert v.table.numel() == 2 and v.num_tokens == 20
    assert np.asarray(c.k.shape).tolist() == [2, 12, 2, 16, 64]
    assert np.asarray(c.v.shape).tolist() == [2, 12, 2, 64, 16]


@pytest.mark.parametrize("D", [32, 64, 128])
def test_k_block_helpers_match_the_oracle_layout(D):
    """The product's torch helpers and the oracle's numpy restatement of the K
    block order agree, and rows -> blocks -> rows is the identity."""
    import torch
    from oracle import attention as oatt
    from rngd_pd_amd.engines.paged_cache import k_block_index, k_block_rows, k_block_tiled
    np.testing.assert_array_equal(k_block_index(D).numpy(), oatt.k_block_index(D))
    rows = torch.randint(-2**15, 2**15, (3, 2, 16, D), dtype=torch.int16)
    blocks = k_block_tiled(rows)
    np.testing.assert_array_equal(blocks.numpy(), oatt.k_block_tiled(rows.numpy()))
    assert torch.equal(k_block_rows(blocks), rows)
