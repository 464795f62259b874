"""A block loaded from a GGUF file (the artifact's record names, dims and widths, at the model's
geometry) runs through the library with the same bits as the same weights built in memory."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_block_from_gguf_records_matches_in_memory_weights(pkg, layer_artifact, dev, tmp_path):
    G, abi = pkg.gguf, pkg.abi
    lw, _ = layer_artifact
    norm = pkg.synth.make_norm_weight(seed=77, device=dev)
    p = tmp_path / "artifact_block.gguf"
    G.write_gguf(str(p), G.layer_records(17, lw, norm), {"general.architecture": "qwen35moe"})
    gf = G.GgufFile(str(p))
    got, gnorm = G.layer_weights(gf, 17, device=dev)
    gf.close()
    p.unlink()
    assert got.up_q is not None and got.down_fmt == lw.down_fmt and got.shared_fmt == lw.shared_fmt
    # the fixture's Zipf logit bias is the synthetic routing skew, not a record of the artifact
    got.router_bias = lw.router_bias
    for T in (1, 64):
        x = pkg.synth.make_input(T, seed=70 + T, device=dev)
        a = abi.block_forward(x, lw, norm_w=norm, residual=x, stages={"topk_ids"})
        b = abi.block_forward(x, got, norm_w=gnorm, residual=x, stages={"topk_ids"})
        torch.cuda.synchronize()
        assert torch.equal(a["topk_ids"].cpu(), b["topk_ids"].cpu()), T
        assert torch.equal(a["combined_out"].cpu().view(torch.int32),
                           b["combined_out"].cpu().view(torch.int32)), T
