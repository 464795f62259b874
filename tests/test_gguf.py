"""GGUF tensor-record ingestion (qwen3.6-35b-a3b_amd/gguf.py) on files this test writes itself:
header, metadata, aligned data start, per-expert byte ranges, the block's records mapped to
LayerWeights in their stored widths, and the refusals (tools/gguf_reader.py:492-620,
engine/loader.py:338-390)."""
import struct

import pytest
import torch


@pytest.fixture(scope="module")
def small_layer(pkg):
    """An artifact-width block at a small geometry (F32 router and scalar gate, separate Q4_K gate
    and up records, Q5_K down, Q8_0 shared expert), on the CPU."""
    Q = pkg.quant
    lw = pkg.synth.make_layer(seed=4, device="cpu", n_experts=16, hidden=256, i_e=256, i_s=256,
                              down_fmt=Q.FMT_Q5_K, router_dtype=torch.float32,
                              scalar_gate_dtype=torch.float32, split_gate_up=True,
                              shared_fmt=Q.FMT_Q8_0)
    norm = pkg.synth.make_norm_weight(seed=4, device="cpu", hidden=256)
    return lw, norm


def _raw(t):
    return t.contiguous().view(torch.uint8)


def test_round_trip_of_a_block(pkg, small_layer, tmp_path):
    G = pkg.gguf
    lw, norm = small_layer
    p = tmp_path / "blk.gguf"
    meta = {"general.architecture": "qwen35moe", "general.name": "synthetic", "x.count": 40,
            "x.eps": 1e-6, "x.flag": True, "x.list": [1, 2, 3]}
    G.write_gguf(str(p), G.layer_records(7, lw, norm), meta, alignment=64)
    gf = G.GgufFile(str(p))
    assert gf.version == 3 and gf.alignment == 64 and gf.data_start % 64 == 0
    assert gf.meta["general.architecture"] == "qwen35moe" and gf.meta["x.count"] == 40
    assert gf.meta["x.flag"] is True and gf.meta["x.list"] == [1, 2, 3]
    assert abs(gf.meta["x.eps"] - 1e-6) < 1e-12
    got, gnorm = G.layer_weights(gf, 7, device="cpu")
    for f in ("router", "gate_up_q", "up_q", "down_q", "shared_gate", "shared_up", "shared_down",
              "shared_scalar_gate"):
        a, b = getattr(got, f), getattr(lw, f)
        assert a.dtype == b.dtype and a.shape == b.shape, f
        assert torch.equal(_raw(a), _raw(b)), f
    assert (got.gate_up_fmt, got.down_fmt, got.shared_fmt) == (lw.gate_up_fmt, lw.down_fmt, lw.shared_fmt)
    assert torch.equal(gnorm, norm)
    gf.close()


def test_fused_gate_up_record(pkg, tmp_path):
    """One ffn_gate_up_exps record [H, 2I, E] (gate rows first) maps to the fused layout."""
    G = pkg.gguf
    lw = pkg.synth.make_layer(seed=5, device="cpu", n_experts=8, hidden=256, i_e=256, i_s=256)
    p = tmp_path / "fused.gguf"
    G.write_gguf(str(p), G.layer_records(0, lw))
    got, norm = G.layer_weights(G.GgufFile(str(p)), 0, device="cpu")
    assert got.up_q is None and norm is None
    assert torch.equal(_raw(got.gate_up_q), _raw(lw.gate_up_q))
    assert got.router.dtype == torch.bfloat16


def test_expert_range_is_the_expert_slab(pkg, small_layer, tmp_path):
    G = pkg.gguf
    lw, norm = small_layer
    p = tmp_path / "r.gguf"
    G.write_gguf(str(p), G.layer_records(2, lw, norm))
    gf = G.GgufFile(str(p))
    data = p.read_bytes()
    for role, t in (("ffn_down_exps", lw.down_q), ("ffn_gate_exps", lw.gate_up_q), ("ffn_up_exps", lw.up_q)):
        for e in (0, 5, 15):
            r = gf.expert_range(G.record_name(2, role), e)
            assert r["length"] == t[e].numel() and r["n_slices"] == 16
            assert data[r["file_off"]:r["file_off"] + r["length"]] == _raw(t[e]).numpy().tobytes()
    with pytest.raises(pkg.Refused, match="expert-index"):
        gf.expert_range(G.record_name(2, "ffn_down_exps"), 16)
    with pytest.raises(pkg.Refused, match="not-routed"):
        gf.expert_range(G.record_name(2, "ffn_gate_inp"), 0)
    with pytest.raises(pkg.Refused, match="unknown-tensor"):
        gf.expert_range("blk.3.ffn_down_exps.weight", 0)


def _header(records, n_kv=0):
    """A bare v3 header with the given (name, dims, type, offset) tensor infos."""
    h = b"GGUF" + struct.pack("<IQQ", 3, len(records), n_kv)
    for name, dims, tid, off in records:
        nb = name.encode()
        h += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        h += struct.pack("<%dQ" % len(dims), *dims) + struct.pack("<IQ", tid, off)
    return h


@pytest.mark.parametrize("case,tag", [
    ("magic", "not-gguf"), ("truncated", "truncated-header"), ("past_eof", "truncated-data"),
    ("misaligned", "misaligned-tensor"), ("duplicate", "duplicate-tensor"), ("version", "gguf-version")])
def test_header_refusals(pkg, tmp_path, case, tag):
    G = pkg.gguf
    rec = ("blk.0.ffn_down_exps.weight", (256, 4, 2), G.GGML_Q4_K, 0)     # 2 x 4 rows x 144 B
    body = _header([rec])
    pad = b"\0" * (-len(body) % 32) + b"\0" * (2 * 4 * 144)
    blob = {"magic": b"GGUX" + (body + pad)[4:], "truncated": body[:-5],
            "past_eof": body + pad[:-1], "misaligned": _header([rec[:3] + (16,)]) + pad + b"\0" * 64,
            "duplicate": _header([rec, rec]) + pad + b"\0" * 2048,
            "version": b"GGUF" + struct.pack("<I", 1) + (body + pad)[8:]}[case]
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(blob)
    with pytest.raises(pkg.Refused, match=tag):
        G.GgufFile(str(p))


def test_role_width_refused(pkg, small_layer, tmp_path):
    """A shared expert stored in a width the kernels do not read (here Q5_K) is refused by name."""
    G = pkg.gguf
    lw, norm = small_layer
    recs = G.layer_records(1, lw, norm)
    fake = [(n, d, (G.GGML_Q4_K if n.endswith("ffn_gate_shexp.weight") else t),
             (b"\0" * G.record_bytes(G.GGML_Q4_K, d[0] * d[1]) if n.endswith("ffn_gate_shexp.weight") else b))
            for n, d, t, b in recs]
    p = tmp_path / "w.gguf"
    G.write_gguf(str(p), fake)
    with pytest.raises(pkg.Refused, match="role-width"):
        G.layer_weights(G.GgufFile(str(p)), 1, device="cpu")
