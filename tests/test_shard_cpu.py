"""Block-aligned sharding of a tensor's elements (host logic of the one-GPU share measured by
bench.py --shard-of): pieces cover the tensor, start on quant-block boundaries, are balanced by
whole blocks, and the views of shard_states address exactly those elements and blocks."""
import pytest
import torch

import mdq_hip


@pytest.mark.parametrize("numel", [0, 1, 127, 128, 129, 1000, 128 * 8, 128 * 8 + 5, 10 ** 6 + 3])
@pytest.mark.parametrize("B,world", [(128, 1), (128, 3), (128, 8), (64, 8), (2048, 4), (1, 5)])
def test_ranges_cover_and_align(numel, B, world):
    r = mdq_hip.block_aligned_ranges(numel, B, world)
    Bc = min(B, 1024)
    assert len(r) == world and r[0][0] == 0 and r[-1][1] == numel
    for (s, e), (s2, _e2) in zip(r, r[1:]):
        assert e == s2
    sizes = []
    for s, e in r:
        assert s <= e and (s == e or s % Bc == 0)          # empty trailing pieces sit at numel
        sizes.append((e - s + Bc - 1) // Bc)
    nb = (numel + Bc - 1) // Bc
    assert sum(sizes) == nb and max(sizes) - min(sizes) <= 1


def test_shard_views_address_their_elements_and_blocks():
    n, B = 1000, 128
    nb = (n + B - 1) // B
    e = mdq_hip.TensorState(torch.arange(n, dtype=torch.float32), torch.arange(n, dtype=torch.float32),
                            torch.arange(n).to(torch.uint8), torch.empty(0, dtype=torch.uint8),
                            torch.arange(nb, dtype=torch.float32), torch.zeros(nb), torch.zeros(nb),
                            3, 4, 1e-3, 0.9, 0.999, 1e-8, 0.01, 7)
    pieces = [mdq_hip.shard_states([e], B, 3, k) for k in range(3)]
    assert [len(x) for x in pieces] == [1, 1, 1]
    got = torch.cat([x[0].p for x in pieces])
    assert torch.equal(got, e.p)
    assert torch.equal(torch.cat([x[0].scale_m for x in pieces]), e.scale_m)
    for x in pieces:
        assert x[0].p.data_ptr() == e.p.data_ptr() + 4 * int(x[0].p[0]) and x[0].tensor_id == 7 and x[0].step == 3
    assert mdq_hip.shard_states([e], B, 16, 15) == []       # 8 blocks over 16 ranks: rank 15 empty
