"""The C-ABI library loads, exports every symbol the header declares, and refuses bad arguments
before touching a device (no GPU needed)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_gfx950.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound(pkg):
    lib = ctypes.CDLL(str(pkg._lib.LIB_PATH))
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(pkg._lib.SIGNATURES), set(names) ^ set(pkg._lib.SIGNATURES)


def test_binding_arity_matches_header(pkg):
    """Each ctypes signature has as many parameters as the header's prototype."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, args) in pkg._lib.SIGNATURES.items():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", text)
        assert m, name
        params = [q for q in m.group(1).split(",") if q.strip() and q.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def test_layer_struct_matches_header(pkg):
    """moe_layer_weights field order and kinds match the ctypes Structure."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct moe_layer_weights\s*\{(.*?)\}", text, re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        kind = "int" if re.match(r"int\b", decl) else "ptr"
        for nm in decl.split(","):
            fields.append((re.sub(r"[^A-Za-z0-9_]", " ", nm).split()[-1], kind))
    got = [(n, "int" if t is ctypes.c_int else "ptr") for n, t in pkg._lib.LayerWeightsC._fields_]
    assert fields == got


def test_abi_version_and_enums_match_header(pkg):
    text = HEADER.read_text()
    assert pkg._lib.lib.moe_abi_version() == int(re.search(r"MOE_ABI_VERSION (\d+)", text).group(1))
    for name in ("MOE_OK", "MOE_E_ARG", "MOE_E_FORMAT", "MOE_E_HIP", "MOE_E_WORKSPACE",
                 "MOE_E_UNSUPPORTED", "MOE_DT_F32", "MOE_DT_BF16", "MOE_FMT_Q4_K", "MOE_FMT_Q5_K", "MOE_FMT_Q6_K",
                 "MOE_FMT_BF16", "MOE_PATH_AUTO", "MOE_PATH_GEMV", "MOE_PATH_MFMA",
                 "MOE_PATH_MFMA_BF16", "MOE_PATH_GEMV_MULTI"):
        m = re.search(name + r"\s*=\s*(-?\d+)", text)
        assert m and int(m.group(1)) == getattr(pkg._lib, name), name


def test_status_words_match_header_and_library(pkg):
    """The status word, test-hook word and status bits of the header, and the router's counter
    index of the library's internal header, as the Python layer uses them."""
    L = pkg._lib
    text = HEADER.read_text()
    for name, attr in (("MOE_STATUS_WORD", "STATUS_WORD"), ("MOE_TEST_HOOK_WORD", "TEST_HOOK_WORD"),
                       ("MOE_STATUS_SPIN_TIMEOUT", "STATUS_SPIN_TIMEOUT"),
                       ("MOE_STATUS_SYNC_STATE", "STATUS_SYNC_STATE")):
        m = re.search(r"#define " + name + r" (\d+)", text)
        assert m and int(m.group(1)) == getattr(L, attr), name
    internal = (ROOT / "qwen3.6-35b-a3b_amd" / "csrc" / "moe_internal.h").read_text()
    assert int(re.search(r"kRouterCntWord = (\d+)", internal).group(1)) == L.ROUTER_CNT_WORD
    assert 4 * (L.ROUTER_CNT_WORD + 256 + 16) <= L.SYNC_BYTES


def test_workspace_bytes_is_monotone(pkg):
    f = pkg._lib.lib.moe_workspace_bytes
    a = f(1, 2048, 512, 256, 8, 512)
    b = f(64, 2048, 512, 256, 8, 512)
    c = f(4096, 2048, 512, 256, 8, 512)
    assert 0 < a < b < c
    # y [T*K, H] f32 dominates at prefill sizes
    assert c >= 4096 * 8 * 2048 * 4
    assert f(0, 2048, 512, 256, 8, 512) == 0


def test_refusals_happen_on_the_host(pkg):
    lib = pkg._lib.lib
    # NULL pointers -> MOE_E_ARG with a message, no device call made
    assert lib.moe_dequant(None, 12, 256, None, 0, None) == pkg._lib.MOE_E_ARG
    assert b"NULL" in lib.moe_last_error()
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.moe_dequant(p, 12, 100, p, 0, None) == pkg._lib.MOE_E_ARG       # not a multiple of 256
    assert lib.moe_dequant(p, 12, 256, p, 5, None) == pkg._lib.MOE_E_ARG       # bad out dtype
    # geometry refusals
    rc = lib.moe_router_topk(p, 0, p, 1, None, 1, 2048, 256, 2, p, None, p, p, p, None, 0, None)
    assert rc == pkg._lib.MOE_E_UNSUPPORTED                                  # K*64 <= E
    assert b"K*64 > E" in lib.moe_last_error()
    rc = lib.moe_block_forward(p, 0, 1, 2048, 512, 256, 8, 512, None, 1e-6, p, None, p, 12, p, 12,
                               p, p, p, p, 0, None, p, None, None, None, None, None, None, None,
                               None, p, 16, None)
    assert rc == pkg._lib.MOE_E_WORKSPACE
    # a negative norm eps is refused before anything else is looked at
    rc = lib.moe_block_forward(p, 0, 1, 2048, 512, 256, 8, 512, p, -1.0, p, None, p, 12, p, 12,
                               p, p, p, p, 0, None, p, None, None, None, None, None, None, None,
                               None, p, 1 << 30, None)
    assert rc == pkg._lib.MOE_E_ARG
    rc = lib.moe_experts(p, 0, p, None, 99, p, 12, p, p, p, 1, 2048, 512, 256, 8, 0, p, p, 1 << 20,
                         None)
    assert rc == pkg._lib.MOE_E_FORMAT
    # the router and the scalar shared gate are bf16 or f32; the shared expert bf16
    rc = lib.moe_router_topk(p, 0, p, 7, None, 1, 2048, 256, 8, p, None, p, p, p, p, 1 << 20, None)
    assert rc == pkg._lib.MOE_E_FORMAT
    rc = lib.moe_shared_expert(p, 0, p, p, p, 12, p, 1, 1, 2048, 512, 0, p, p, p, 1 << 20, None)
    assert rc == pkg._lib.MOE_E_FORMAT
    rc = lib.moe_shared_expert(p, 0, p, p, p, 30, p, 7, 1, 2048, 512, 0, p, p, p, 1 << 20, None)
    assert rc == pkg._lib.MOE_E_FORMAT
    # the descriptor entry checks the descriptor's formats the same way
    L = pkg._lib
    W = L.LayerWeightsC(p.value, 7, None, p.value, None, 12, p.value, 13, p.value, p.value,
                        p.value, 30, p.value, 0, p.value)
    rc = lib.moe_block_forward_w(p, 0, 1, 2048, 512, 256, 8, 512, ctypes.byref(W), 1e-6, 0, None,
                                 p, None, None, None, None, None, None, None, None, p, 1 << 30,
                                 None, None)
    assert rc == pkg._lib.MOE_E_FORMAT
    W.router_dtype = 0
    W.down_fmt = 99
    rc = lib.moe_block_forward_w(p, 0, 1, 2048, 512, 256, 8, 512, ctypes.byref(W), 1e-6, 0, None,
                                 p, None, None, None, None, None, None, None, None, p, 1 << 30,
                                 None, None)
    assert rc == pkg._lib.MOE_E_FORMAT
    rc = lib.moe_block_forward_w(p, 0, 1, 2048, 512, 256, 8, 512, None, 1e-6, 0, None,
                                 p, None, None, None, None, None, None, None, None, p, 1 << 30,
                                 None, None)
    assert rc == pkg._lib.MOE_E_ARG
    assert lib.moe_workspace_init(p, 16, None) == pkg._lib.MOE_E_ARG
    # the sort's scratch starts after the sync words: a workspace that only holds the scratch
    # itself is too small
    # 512 KiB + 256 experts x 1 chunk count padded to 4 x 4 B
    rc = lib.moe_sort_permute(p, 16, 8, 256, p, p, p, p, p, 4096, None)
    assert rc == pkg._lib.MOE_E_WORKSPACE and b"528384" in lib.moe_last_error()


def test_product_path_never_imports_the_oracle():
    """The package must not import, call or fall back to anything under oracle/."""
    for f in (ROOT / "qwen3.6-35b-a3b_amd").rglob("*.py"):
        src = f.read_text()
        assert "oracle" not in re.sub(r'""".*?"""', "", src, flags=re.S), f
