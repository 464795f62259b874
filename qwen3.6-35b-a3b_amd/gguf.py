"""GGUF tensor records -> one MoE block's device weights (the layout `moe_layer_weights` names).

Written from the GGUF container format (v2 / v3, little endian):
  header   "GGUF" | u32 version | u64 n_tensors | u64 n_kv
  n_kv     key (u64 length + utf-8) | u32 value type | value   (type 9 = array: u32 type, u64 n, n values)
  n_tensors name | u32 n_dims | u64 dims[n_dims] (dims[0] the fastest axis) | u32 ggml type | u64 offset
  data     starts at the header's end rounded up to `general.alignment` (32 when absent); each
           record's offset is relative to it and a multiple of the alignment.

A routed-expert record (`blk.N.ffn_{gate,up,down}_exps.weight`) has dims [cols, rows, E]: the expert
axis is the slowest, so expert e is the contiguous byte range [e * L, (e + 1) * L) of the record with
L = rows * cols / block_elts * block_bytes, exactly the [E][rows][blocks] layout the kernels read.

Replaces tools/gguf_reader.py:492-620 (`Gguf`: header parse, data windows) and
engine/loader.py:338-390 (`expert_range`) for the MoE block's records; `layer_weights` is what the
layer loop's `E.read(role, layer)` / `E.expert(...)` (engine/m3_forward.py:235-283) collect for one
block, uploaded once in the stored widths instead of decoded to f32 on every read. Every refusal is
`abi.Refused(tag, message)`.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

# ggml type id -> (elements per block, bytes per block) for the widths this block can hold
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_BF16 = 0, 1, 8, 12, 13, 14, 30
BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144),
         GGML_Q5_K: (256, 176), GGML_Q6_K: (256, 210), GGML_BF16: (1, 2)}
TYPE_NAMES = {GGML_F32: "F32", GGML_F16: "F16", GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K",
              GGML_Q5_K: "Q5_K", GGML_Q6_K: "Q6_K", GGML_BF16: "BF16"}

# Metadata value types of the container: type id -> numpy dtype of one element (little endian).
# 8 (a length-prefixed string) and 9 (a typed, counted array) carry their own lengths.
_META_DTYPE = {0: np.dtype("<u1"), 1: np.dtype("<i1"), 2: np.dtype("<u2"), 3: np.dtype("<i2"),
               4: np.dtype("<u4"), 5: np.dtype("<i4"), 6: np.dtype("<f4"), 7: np.dtype("?"),
               10: np.dtype("<u8"), 11: np.dtype("<i8"), 12: np.dtype("<f8")}
GGUF_STRING, GGUF_ARRAY = 8, 9
_U32, _U64 = np.dtype("<u4"), np.dtype("<u8")
LIST_MAX = 4096            # numeric arrays up to this length become lists, longer ones stay arrays


def _refused(tag: str, msg: str):
    from .abi import Refused
    return Refused(tag, msg)


def record_bytes(type_id: int, n_elts: int) -> int:
    """Stored bytes of n_elts elements of a ggml type (whole blocks only)."""
    if type_id not in BLOCK:
        raise _refused("unsupported-type", f"ggml type {type_id} is not one this block reads")
    qk, bb = BLOCK[type_id]
    if n_elts % qk:
        raise _refused("partial-block", f"{n_elts} elements are not whole {TYPE_NAMES[type_id]} blocks of {qk}")
    return n_elts // qk * bb


def _round_up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


@dataclass(frozen=True)
class GgufTensor:
    index: int
    name: str
    dims: tuple           # GGUF order: dims[0] is the fastest axis
    type_id: int
    offset: int           # bytes from the start of the data section
    nbytes: int

    @property
    def shape_hf(self) -> tuple:
        """The record's shape with the slowest axis first (HF / torch order)."""
        return self.dims[::-1]

    @property
    def type_name(self) -> str:
        return TYPE_NAMES.get(self.type_id, f"type_{self.type_id}")


class _HeaderCursor:
    """A forward-only position in the mapped file. Every field is decoded in place from the
    memoryview (numpy views of the bytes, no reads through a file object); a field that would run
    past the end of the file is refused with its name and position."""

    __slots__ = ("buf", "pos", "path")

    def __init__(self, buf: memoryview, path: str):
        self.buf, self.pos, self.path = buf, 0, path

    def claim(self, n: int, what: str) -> int:
        """Start of the next n bytes, which now belong to `what`."""
        at = self.pos
        if n < 0 or at + n > len(self.buf):
            raise _refused("truncated-header", f"{self.path}: the {what} at byte {at} needs {n} bytes; "
                                               f"the file ends at byte {len(self.buf)}")
        self.pos = at + n
        return at

    def array(self, dt: np.dtype, count: int, what: str) -> np.ndarray:
        at = self.claim(dt.itemsize * count, what)
        return np.frombuffer(self.buf, dtype=dt, count=count, offset=at)

    def u32(self, what: str) -> int:
        return int(self.array(_U32, 1, what)[0])

    def u64(self, what: str) -> int:
        return int(self.array(_U64, 1, what)[0])

    def text(self, what: str) -> str:
        n = self.u64(f"length of the {what}")
        at = self.claim(n, what)
        return bytes(self.buf[at:at + n]).decode("utf-8", "replace")

    def meta_value(self, vt: int, key: str):
        if vt == GGUF_STRING:
            return self.text(f"string value of {key!r}")
        if vt == GGUF_ARRAY:
            et = self.u32(f"element type of {key!r}")
            n = self.u64(f"element count of {key!r}")
            dt = _META_DTYPE.get(et)
            if dt is not None:
                vals = self.array(dt, n, f"array value of {key!r}")
                return vals.tolist() if n <= LIST_MAX else vals
            return [self.meta_value(et, key) for _ in range(n)]
        dt = _META_DTYPE.get(vt)
        if dt is None:
            raise _refused("bad-header", f"{self.path}: metadata {key!r} has value type {vt}, "
                                         "which the container does not define")
        return self.array(dt, 1, f"value of {key!r}")[0].item()


class GgufFile:
    """A GGUF file mapped read-only once: the header is decoded in place from the map (nothing of
    the data section is touched), and record bytes are views of the same map."""

    def __init__(self, path: str):
        self.path = str(path)
        self.size = os.path.getsize(self.path)
        if self.size < 4:
            raise _refused("not-gguf", f"{self.path}: {self.size} bytes, shorter than the magic")
        with open(self.path, "rb") as fh:
            self._mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        self._buf = memoryview(self._mm)
        self._read_header(_HeaderCursor(self._buf, self.path))

    # ------------------------------------------------------------------------------ header --
    def _read_header(self, cur: _HeaderCursor) -> None:
        if bytes(self._buf[:4]) != b"GGUF":
            raise _refused("not-gguf", f"{self.path}: the first bytes are {bytes(self._buf[:4])!r}, not b'GGUF'")
        cur.claim(4, "magic")
        self.version = cur.u32("version")
        if self.version not in (2, 3):
            raise _refused("gguf-version", f"{self.path}: container version {self.version}; "
                                           "versions 2 and 3 are read")
        n_tensors = cur.u64("tensor count")
        n_kv = cur.u64("metadata count")
        self.meta: dict = {}
        for _ in range(n_kv):
            key = cur.text("metadata key")
            self.meta[key] = cur.meta_value(cur.u32(f"value type of {key!r}"), key)
        self.tensors: list[GgufTensor] = []
        self.by_name: dict[str, GgufTensor] = {}
        for i in range(n_tensors):
            name = cur.text(f"name of tensor {i}")
            nd = cur.u32(f"rank of {name!r}")
            if nd < 1 or nd > 4:
                raise _refused("bad-header", f"{self.path}: {name!r} claims {nd} axes (1 to 4 exist)")
            dims = tuple(int(d) for d in cur.array(_U64, nd, f"axes of {name!r}"))
            tid = cur.u32(f"ggml type of {name!r}")
            off = cur.u64(f"data offset of {name!r}")
            n_elts = 1
            for d in dims:
                n_elts *= d
            rec = GgufTensor(i, name, dims, tid, off, record_bytes(tid, n_elts) if tid in BLOCK else -1)
            if name in self.by_name:
                raise _refused("duplicate-tensor", f"{self.path}: tensor {name!r} is listed twice "
                                                   f"(entries {self.by_name[name].index} and {i})")
            self.by_name[name] = rec
            self.tensors.append(rec)
        self.header_end = cur.pos
        align = self.meta.get("general.alignment", 32)
        if not isinstance(align, int) or align <= 0:
            raise _refused("bad-header", f"{self.path}: general.alignment = {align!r}")
        self.alignment = align
        self.data_start = _round_up(self.header_end, align)
        for t in self.tensors:
            if t.offset % align:
                raise _refused("misaligned-tensor", f"{t.name}: data offset {t.offset} is off the "
                                                    f"{align}-byte grid")
            if t.nbytes >= 0 and self.data_start + t.offset + t.nbytes > self.size:
                raise _refused("truncated-data", f"{t.name}: its {t.nbytes} bytes at data offset "
                                                 f"{t.offset} end past byte {self.size} of {self.path}")

    # --------------------------------------------------------------------------- records --
    def tensor(self, name: str) -> GgufTensor:
        t = self.by_name.get(name)
        if t is None:
            raise _refused("unknown-tensor", f"{name!r} is not in {self.path}")
        if t.nbytes < 0:
            raise _refused("unsupported-type", f"{name} stores ggml type {t.type_id}")
        return t

    def view(self, name: str) -> np.ndarray:
        """The record's bytes, a read-only uint8 view of the mapped file (no copy)."""
        t = self.tensor(name)
        return np.frombuffer(self._buf, dtype=np.uint8, count=t.nbytes,
                             offset=self.data_start + t.offset)

    def expert_range(self, name: str, idx: int) -> dict:
        """Expert `idx`'s contiguous byte range in a routed record (engine/loader.py:338-390), or a
        refusal naming the reason: not a 3-axis record, an expert index outside [0, E), a slice
        that splits a quantized block, or an expert axis that does not tile the record."""
        t = self.tensor(name)
        if len(t.dims) != 3:
            raise _refused("not-routed", f"{name} has dims {t.dims}: no expert axis")
        e = int(t.dims[2])
        if e <= 1:
            raise _refused("not-an-expert-axis", f"{name}: the slowest axis is {e} wide")
        idx = int(idx)
        if not 0 <= idx < e:
            raise _refused("expert-index", f"{name}: expert {idx} is outside [0, {e})")
        inner = int(t.dims[0]) * int(t.dims[1])
        qk, bb = BLOCK[t.type_id]
        if inner % qk or int(t.dims[0]) % qk:
            raise _refused("expert-slice-splits-block", f"{name}: a row of {t.dims[0]} elements is not "
                                                        f"whole {t.type_name} blocks of {qk}")
        length = inner // qk * bb
        if length * e != t.nbytes:
            raise _refused("expert-axis-does-not-tile", f"{name}: {e} slices of {length} B != {t.nbytes} B")
        return dict(name=name, index=idx, n_slices=e, file_off=self.data_start + t.offset + idx * length,
                    length=length, elts=inner, type_name=t.type_name)

    def close(self) -> None:
        """Release the map. Views returned by `view` keep it alive until they are collected."""
        if self._buf is not None:
            self._buf.release()
            self._buf = None
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass
            self._mm = None


# ------------------------------------------------------------------------- one MoE block --
# the block's records (engine/m3_forward.py:203-211 name_for: blk.<layer>.<role>.weight)
ROUTER, SCALAR_GATE = "ffn_gate_inp", "ffn_gate_inp_shexp"
SHARED = ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")
GATE, UP, GATE_UP, DOWN = "ffn_gate_exps", "ffn_up_exps", "ffn_gate_up_exps", "ffn_down_exps"
NORM = "post_attention_norm"


def record_name(layer: int, role: str) -> str:
    return f"blk.{layer}.{role}.weight"


def _want(gf: GgufFile, name: str, dims: tuple, types: tuple) -> GgufTensor:
    t = gf.tensor(name)
    if tuple(int(d) for d in t.dims) != tuple(dims):
        raise _refused("shape", f"{name}: dims {t.dims}, expected {dims} (GGUF order)")
    if t.type_id not in types:
        raise _refused("role-width", f"{name} stores {t.type_name}; this block reads "
                                     + " / ".join(TYPE_NAMES[x] for x in types))
    return t


def layer_weights(gf: GgufFile, layer: int, device="cuda", top_k: int = 8):
    """Block `layer`'s MoE weights as a weights.LayerWeights on `device`, each record uploaded in
    its stored width (the artifact: F32 router and scalar gate, Q4_K gate and up, Q5_K / Q6_K
    down, Q8_0 shared expert), plus the post-attention norm weight (f32 [H], the stored 1 + w) or
    None when the file has none. Gate and up come from separate records, or from one fused
    `ffn_gate_up_exps` record (gate rows first)."""
    import torch

    from . import quant as Q
    from .weights import LayerWeights

    dev = torch.device(device)
    rn = lambda role: record_name(layer, role)

    def upload(name: str, shape: tuple, dtype=torch.uint8) -> torch.Tensor:
        raw = torch.from_numpy(gf.view(name).copy())
        if dtype is not torch.uint8:
            raw = raw.view(dtype)
        return raw.reshape(shape).to(dev)

    r = gf.tensor(rn(ROUTER))
    if len(r.dims) != 2:
        raise _refused("shape", f"{rn(ROUTER)}: dims {r.dims}")
    H, E = int(r.dims[0]), int(r.dims[1])
    _want(gf, rn(ROUTER), (H, E), (GGML_F32, GGML_BF16))
    rdt = torch.float32 if r.type_id == GGML_F32 else torch.bfloat16
    router = upload(rn(ROUTER), (E, H), rdt)

    expert_types = (GGML_Q4_K, GGML_Q6_K, GGML_BF16)
    if rn(GATE_UP) in gf.by_name:
        gu = gf.tensor(rn(GATE_UP))
        two_i = int(gu.dims[1])
        _want(gf, rn(GATE_UP), (H, two_i, E), expert_types)
        gate_up = upload(rn(GATE_UP), (E, two_i, Q.row_bytes(gu.type_id, H)))
        up_q, I, gu_fmt = None, two_i // 2, gu.type_id
    else:
        g = gf.tensor(rn(GATE))
        I = int(g.dims[1])
        _want(gf, rn(GATE), (H, I, E), expert_types)
        _want(gf, rn(UP), (H, I, E), (g.type_id,))
        gate_up = upload(rn(GATE), (E, I, Q.row_bytes(g.type_id, H)))
        up_q = upload(rn(UP), (E, I, Q.row_bytes(g.type_id, H)))
        gu_fmt = g.type_id
    d = _want(gf, rn(DOWN), (I, H, E), (GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_BF16))
    down = upload(rn(DOWN), (E, H, Q.row_bytes(d.type_id, I)))

    sg = gf.tensor(rn(SHARED[0]))
    Is = int(sg.dims[1])
    s_types = (GGML_Q8_0, GGML_BF16)
    _want(gf, rn(SHARED[0]), (H, Is), s_types)
    _want(gf, rn(SHARED[1]), (H, Is), (sg.type_id,))
    _want(gf, rn(SHARED[2]), (Is, H), (sg.type_id,))
    if sg.type_id == GGML_Q8_0:
        sfmt = Q.FMT_Q8_0
        shared = [upload(rn(SHARED[0]), (Is, H // 32 * 34)), upload(rn(SHARED[1]), (Is, H // 32 * 34)),
                  upload(rn(SHARED[2]), (H, Is // 32 * 34))]
    else:
        sfmt = Q.FMT_BF16
        shared = [upload(rn(SHARED[0]), (Is, H), torch.bfloat16), upload(rn(SHARED[1]), (Is, H), torch.bfloat16),
                  upload(rn(SHARED[2]), (H, Is), torch.bfloat16)]
    sgt = gf.tensor(rn(SCALAR_GATE))
    if tuple(int(x) for x in sgt.dims) not in ((H,), (H, 1)) or sgt.type_id not in (GGML_F32, GGML_BF16):
        raise _refused("shape", f"{rn(SCALAR_GATE)}: dims {sgt.dims} type {sgt.type_name}")
    scalar_gate = upload(rn(SCALAR_GATE), (1, H), torch.float32 if sgt.type_id == GGML_F32 else torch.bfloat16)

    norm = None
    if rn(NORM) in gf.by_name:
        _want(gf, rn(NORM), (H,), (GGML_F32,))
        norm = upload(rn(NORM), (H,), torch.float32)

    lw = LayerWeights(router=router, gate_up_q=gate_up, gate_up_fmt=gu_fmt, down_q=down,
                      down_fmt=d.type_id, shared_gate=shared[0], shared_up=shared[1],
                      shared_down=shared[2], shared_scalar_gate=scalar_gate, top_k=top_k,
                      up_q=up_q, shared_fmt=sfmt)
    lw.validate()
    return lw, norm


# --------------------------------------------------------------------------------- writer --
def write_gguf(path: str, records: list, meta: dict | None = None, alignment: int = 32) -> None:
    """Write a GGUF v3 file: `records` is a list of (name, dims in GGUF order, ggml type id, bytes);
    `meta` maps keys to str / int (u32, or u64 above 2^32) / float (f32) / bool values or lists of
    ints (u32 arrays). For tests and for packing synthetic blocks in the artifact's layout."""
    meta = dict(meta or {})
    if alignment != 32:
        meta["general.alignment"] = alignment

    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    def val(v) -> bytes:
        if isinstance(v, bool):
            return struct.pack("<IB", 7, int(v))
        if isinstance(v, str):
            return struct.pack("<I", GGUF_STRING) + s(v)
        if isinstance(v, float):
            return struct.pack("<If", 6, v)
        if isinstance(v, int):
            return struct.pack("<II", 4, v) if 0 <= v < 2 ** 32 else struct.pack("<Iq", 11, v)
        if isinstance(v, (list, tuple)):
            return struct.pack("<IIQ", GGUF_ARRAY, 4, len(v)) + struct.pack("<%dI" % len(v), *v)
        raise TypeError(f"metadata value {v!r}")

    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(records), len(meta)))
    for k, v in meta.items():
        head += s(k) + val(v)
    offs, off = [], 0
    for name, dims, tid, data in records:
        n = 1
        for d in dims:
            n *= int(d)
        if len(data) != record_bytes(tid, n):
            raise ValueError(f"{name}: {len(data)} bytes for dims {dims} of type {tid}")
        offs.append(off)
        off = -(-(off + len(data)) // alignment) * alignment
    for (name, dims, tid, _), o in zip(records, offs):
        head += s(name) + struct.pack("<I", len(dims)) + struct.pack("<%dQ" % len(dims), *dims)
        head += struct.pack("<IQ", tid, o)
    data_start = -(-len(head) // alignment) * alignment
    with open(path, "wb") as fh:
        fh.write(head)
        fh.write(b"\0" * (data_start - len(head)))
        pos = 0
        for (name, dims, tid, data), o in zip(records, offs):
            fh.write(b"\0" * (o - pos))
            fh.write(bytes(data))
            pos = o + len(data)
        fh.write(b"\0" * (-pos % alignment))


def layer_records(layer: int, lw, norm_w=None) -> list:
    """The GGUF records of one block held as weights.LayerWeights (the inverse of layer_weights):
    the artifact's names, dims in GGUF order, ggml type ids and the stored bytes."""
    import torch

    from . import quant as Q

    def raw(t: torch.Tensor) -> bytes:
        return t.detach().contiguous().cpu().view(torch.uint8).numpy().tobytes()

    E, H = lw.router.shape
    I, Is = lw.i_e, lw.i_s
    f32_or_bf16 = lambda t: GGML_F32 if t.dtype == torch.float32 else GGML_BF16
    rn = lambda role: record_name(layer, role)
    recs = [(rn(ROUTER), (H, E), f32_or_bf16(lw.router), raw(lw.router))]
    if lw.up_q is not None:
        recs += [(rn(GATE), (H, I, E), lw.gate_up_fmt, raw(lw.gate_up_q)),
                 (rn(UP), (H, I, E), lw.gate_up_fmt, raw(lw.up_q))]
    else:
        recs.append((rn(GATE_UP), (H, 2 * I, E), lw.gate_up_fmt, raw(lw.gate_up_q)))
    recs.append((rn(DOWN), (I, H, E), lw.down_fmt, raw(lw.down_q)))
    st = GGML_Q8_0 if lw.shared_fmt == Q.FMT_Q8_0 else GGML_BF16
    recs += [(rn(SHARED[0]), (H, Is), st, raw(lw.shared_gate)),
             (rn(SHARED[1]), (H, Is), st, raw(lw.shared_up)),
             (rn(SHARED[2]), (Is, H), st, raw(lw.shared_down)),
             (rn(SCALAR_GATE), (H,), f32_or_bf16(lw.shared_scalar_gate), raw(lw.shared_scalar_gate))]
    if norm_w is not None:
        recs.append((rn(NORM), (H,), GGML_F32, raw(norm_w.float())))
    return recs
