"""Token->expert grouping is bit-exact vs torch.argsort(ids.flatten(), stable=True)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ids(T, K, E, seed, zipf):
    g = torch.Generator().manual_seed(seed)
    if zipf:
        w = torch.arange(1, E + 1, dtype=torch.float64).pow(-1.1)
        rows = [torch.multinomial(w, K, replacement=False, generator=g) for _ in range(T)]
        return torch.stack(rows).to(torch.int32)
    return torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)


# chunks of 1024 pairs up to 128 chunks (129, 300, 4096, 4097, 16384 tokens: partial last chunks
# at 129, 300, 4097), longer above (20000 tokens: 1280-pair chunks)
@pytest.mark.parametrize("T,zipf", [(1, False), (8, False), (9, True), (64, True), (128, True),
                                    (129, False), (300, False), (4096, False), (4097, True),
                                    (16384, True), (20000, False)])
def test_sort_permute_matches_stable_argsort(pkg, dev, T, zipf):
    K, E = 8, 256
    ids = _ids(T, K, E, seed=T, zipf=zipf)
    gr = pkg.abi.sort_permute(ids.to(dev), E)
    torch.cuda.synchronize()
    flat = ids.flatten().long()
    want = torch.argsort(flat, stable=True)
    assert torch.equal(gr["sorted_pairs"].cpu().long(), want)
    inv = torch.empty_like(want)
    inv[want] = torch.arange(len(want))
    assert torch.equal(gr["pair_pos"].cpu().long(), inv)
    counts = torch.bincount(flat, minlength=E)
    off = torch.zeros(E + 1, dtype=torch.long)
    off[1:] = torch.cumsum(counts, 0)
    assert torch.equal(gr["expert_offsets"].cpu().long(), off)
    hits = torch.unique(flat)
    hl = gr["hit_list"].cpu().long()
    assert hl[0].item() == len(hits)
    assert torch.equal(hl[1:1 + len(hits)], hits)
