"""GGUF ingestion for the MoE decode path: a reader (and a writer, for
fixtures and conversions) of GGUF v2/v3 files, and the mapping of one MoE
layer's tensors onto the stacked device buffers and strides that the fused
layer (``chimere_moe_ffn_decode``) takes.

The reader follows the reference's ``GgufFile`` (cs/src/gguf_loader.rs:298-618):
little-endian header (magic "GGUF", version 2 or 3, u64 tensor and KV
counts), typed metadata KV pairs (value types :42-95, strings as u64 length +
UTF-8 bytes :623-638, arrays as element type + u64 count + values :651-696),
tensor infos (name, u32 n_dims, u64 dims innermost first, u32 ggml type, u64
offset :375-404), and a data section starting at the header end rounded up to
``general.alignment`` (default 32, :367-373, :406-412).  Tensor bytes are
``n_elements / block_elems * block_bytes`` (:161-199), read without copying
from a memory map.  Errors raise ``GgufError`` with the reference's messages.

The MoE tensor names and layouts are those of the reference's loader
(cs/src/qwen35_model/compute_graph.rs:988-1000, 1395-1440):
``blk.{il}.ffn_gate_inp.weight`` router [E, H] f32, ``ffn_{gate,up}_exps``
[E][F rows][H], ``ffn_down_exps`` [E][H rows][F] (all experts contiguous, one
stride per expert), ``ffn_{gate,up,down}_shexp`` the shared expert and
``ffn_gate_inp_shexp`` its sigmoid gate vector [H]; top-k from
``{arch}.expert_used_count`` (cs/src/config.rs:414-421).
"""
import mmap
import os
import struct

import numpy as np

GGUF_MAGIC = 0x46554747          # "GGUF" little-endian
DEFAULT_ALIGNMENT = 32

# metadata value types
(UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY,
 UINT64, INT64, FLOAT64) = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i",
           FLOAT32: "<f", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# ggml tensor types: id -> (elements per block, bytes per block)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ3_S, BF16, MXFP4 = 0, 1, 2, 8, 12, 13, 14, 21, 30, 39
BLOCK_INFO = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 40),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
    16: (256, 66), 17: (256, 74), 18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110),
    22: (256, 82), 23: (256, 136), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
    29: (256, 56), 30: (1, 2), 39: (32, 17),
}


class GgufError(ValueError):
    pass


def tensor_bytes(ggml_type, n_elements):
    e, b = BLOCK_INFO[ggml_type]
    return n_elements * b // e


class TensorInfo:
    def __init__(self, name, dims, ggml_type, data_offset):
        self.name, self.dims, self.ggml_type, self.data_offset = name, tuple(dims), ggml_type, data_offset
        self.n_elements = int(np.prod(self.dims, dtype=np.int64)) if self.dims else 1

    @property
    def nbytes(self):
        return tensor_bytes(self.ggml_type, self.n_elements)

    def __repr__(self):
        return f"TensorInfo({self.name!r}, dims={self.dims}, type={self.ggml_type}, offset={self.data_offset})"


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n, what="value"):
        if self.pos + n > len(self.buf):
            raise GgufError(f"{what} extends beyond file")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def scalar(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        n = self.scalar("<Q")
        try:
            return bytes(self.take(n, "String")).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GgufError(str(e)) from None

    def value(self, vtype):
        if vtype in _SCALAR:
            return self.scalar(_SCALAR[vtype])
        if vtype == BOOL:
            return self.scalar("<B") != 0
        if vtype == STRING:
            return self.string()
        if vtype == ARRAY:
            et = self.scalar("<I")
            if et > FLOAT64:
                raise GgufError(f"Unknown array element type: {et}")
            n = self.scalar("<Q")
            return [self.value(et) for _ in range(n)]
        raise GgufError(f"Unknown GGUF value type: {vtype}")


class GgufFile:
    """A parsed GGUF file; tensor data stays memory-mapped (cs/src/gguf_loader.rs:298-618)."""

    def __init__(self, path):
        self.path = os.fspath(path)
        with open(self.path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if os.path.getsize(self.path) else b""
        buf = memoryview(self._mm)
        c = _Cursor(buf)
        magic = c.scalar("<I")
        if magic != GGUF_MAGIC:
            raise GgufError(f"Invalid GGUF magic: 0x{magic:08X} (expected 0x{GGUF_MAGIC:08X})")
        self.version = c.scalar("<I")
        if self.version < 2 or self.version > 3:
            raise GgufError(f"Unsupported GGUF version: {self.version} (expected 2 or 3)")
        self.n_tensors = c.scalar("<Q")
        self.n_kv = c.scalar("<Q")
        self.metadata, self.metadata_types = {}, {}
        for _ in range(self.n_kv):
            key = c.string()
            vt = c.scalar("<I")
            self.metadata[key] = c.value(vt)
            self.metadata_types[key] = vt
        al = self.metadata.get("general.alignment")
        self.alignment = int(al) if isinstance(al, int) and not isinstance(al, bool) and al > 0 else DEFAULT_ALIGNMENT
        self.tensors, self._index = [], {}
        for i in range(self.n_tensors):
            name = c.string()
            nd = c.scalar("<I")
            dims = [c.scalar("<Q") for _ in range(nd)]
            t = c.scalar("<I")
            if t not in BLOCK_INFO:
                raise GgufError(f"Unknown GGML type {t} for tensor '{name}'")
            off = c.scalar("<Q")
            self._index[name] = i
            self.tensors.append(TensorInfo(name, dims, t, off))
        end = c.pos
        self.data_section_offset = end if end % self.alignment == 0 else end + self.alignment - end % self.alignment
        self._buf = buf

    # -- the reference's accessors
    def get_metadata(self, key):
        return self.metadata.get(key)

    def get_tensor_info(self, name):
        i = self._index.get(name)
        return None if i is None else self.tensors[i]

    def tensor_names(self):
        return [t.name for t in self.tensors]

    def tensor_ggml_type(self, name):
        t = self.get_tensor_info(name)
        return None if t is None else t.ggml_type

    def tensor_data(self, info):
        """Raw bytes of a tensor as a read-only uint8 array (no copy)."""
        if isinstance(info, str):
            name = info
            info = self.get_tensor_info(name)
            if info is None:
                raise GgufError(f"Tensor '{name}' not found in GGUF file")
        start = self.data_section_offset + info.data_offset
        end = start + info.nbytes
        if end > len(self._buf):
            raise GgufError(f"Tensor '{info.name}' data extends beyond file: {start}+{info.nbytes} > {len(self._buf)}")
        return np.frombuffer(self._buf, dtype=np.uint8, count=info.nbytes, offset=start)

    def load_f32(self, name):
        """An F32 / F16 / BF16 tensor as float32, shape = dims reversed (outermost first)."""
        info = self.get_tensor_info(name)
        if info is None:
            raise GgufError(f"Tensor '{name}' not found in GGUF file")
        raw = self.tensor_data(info)
        if info.ggml_type == F32:
            a = raw.view(np.float32)
        elif info.ggml_type == F16:
            a = raw.view(np.float16).astype(np.float32)
        elif info.ggml_type == BF16:
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            raise GgufError(f"Tensor '{name}' is of type {info.ggml_type}, not a float type")
        return a.reshape(tuple(reversed(info.dims)))

    def close(self):
        """Unmaps the file once no array returned by tensor_data is alive."""
        try:
            self._buf.release()
            if hasattr(self._mm, "close"):
                self._mm.close()
        except BufferError:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ------------------------------------------------------------------ writer

def _pack_value(vt, v):
    if vt in _SCALAR:
        return struct.pack(_SCALAR[vt], v)
    if vt == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if vt == STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if vt == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_pack_value(et, x) for x in items)
    raise GgufError(f"Unknown GGUF value type: {vt}")


def write_gguf(path, metadata, tensors, alignment=DEFAULT_ALIGNMENT, version=3):
    """Write a GGUF file.  metadata: {key: (value_type, value)} (arrays as
    (ARRAY, (elem_type, [values]))); tensors: [(name, dims innermost first,
    ggml_type, bytes-like of exactly tensor_bytes(type, prod(dims)))]."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = (UINT32, alignment)
    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(md))
    for k, (vt, v) in md.items():
        head += _pack_value(STRING, k) + struct.pack("<I", vt) + _pack_value(vt, v)
    offs, off = [], 0
    for name, dims, t, data in tensors:
        n = len(memoryview(data).cast("B"))
        if n != tensor_bytes(t, int(np.prod(dims, dtype=np.int64))):
            raise GgufError(f"tensor '{name}': {n} bytes for dims {dims} of type {t}")
        offs.append(off)
        off += n
        off += (-off) % alignment
    for (name, dims, t, _), o in zip(tensors, offs):
        head += _pack_value(STRING, name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", t, o)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (name, dims, t, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            b = bytes(memoryview(data).cast("B"))
            f.write(b)
            pos = o + len(b)


# ------------------------------------------------------- MoE layer mapping

def moe_tensors(g, il):
    """Names, types and shapes of layer il's MoE tensors, checked against each
    other; returns a dict with H, F, E, K and the tensor infos."""
    nm = lambda s: f"blk.{il}.{s}.weight"   # noqa: E731
    req = {k: g.get_tensor_info(nm(k)) for k in ("ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")}
    for k, v in req.items():
        if v is None:
            raise GgufError(f"Tensor '{nm(k)}' not found in GGUF file")
    H, E = req["ffn_gate_inp"].dims
    gd, ud, dd = req["ffn_gate_exps"].dims, req["ffn_up_exps"].dims, req["ffn_down_exps"].dims
    F = gd[1]
    if gd != (H, F, E) or ud != (H, F, E) or dd != (F, H, E):
        raise GgufError(f"layer {il}: expert tensor dims {gd} {ud} {dd} do not match router [{H}, {E}]")
    te = req["ffn_gate_exps"].ggml_type
    if req["ffn_up_exps"].ggml_type != te or req["ffn_down_exps"].ggml_type != te:
        raise GgufError(f"layer {il}: gate/up/down experts of different types")
    sh = [g.get_tensor_info(nm(k)) for k in ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")]
    if any(s is not None for s in sh):
        if any(s is None for s in sh):
            raise GgufError(f"layer {il}: shared expert incomplete")
        if sh[0].dims != (H, F) or sh[1].dims != (H, F) or sh[2].dims != (F, H):
            raise GgufError(f"layer {il}: shared expert dims {sh[0].dims} {sh[1].dims} {sh[2].dims}, "
                            f"expected [{H}, {F}] / [{F}, {H}] (same FFN width as the routed experts)")
        if len({s.ggml_type for s in sh}) != 1:
            raise GgufError(f"layer {il}: shared gate/up/down of different types")
    else:
        sh = None
    gate_vec = g.get_tensor_info(nm("ffn_gate_inp_shexp"))
    arch = g.get_metadata("general.architecture")
    K = g.get_metadata(f"{arch}.expert_used_count") if arch else None
    return {"H": H, "F": F, "E": E, "K": K, "expert_type": te, "tensors": req, "shared": sh,
            "shared_type": sh[0].ggml_type if sh else -1, "gate_vec": gate_vec}


def moe_layer_from_gguf(g, il, device, top_k=None, max_ntok=8):
    """MoeLayer for layer il of GGUF file g, its tensors copied to `device`."""
    import torch

    from .moe import MoeLayer
    m = moe_tensors(g, il)
    K = top_k if top_k is not None else m["K"]
    if not K:
        raise GgufError("top_k not given and no {arch}.expert_used_count in the metadata")
    t = m["tensors"]
    dev = lambda a: torch.from_numpy(np.array(a, copy=True)).to(device)   # noqa: E731
    router = dev(g.load_f32(t["ffn_gate_inp"].name))
    E = m["E"]
    gate, up, down = (dev(g.tensor_data(t[k]).reshape(E, -1)) for k in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"))
    shared = tuple(dev(g.tensor_data(s)) for s in m["shared"]) if m["shared"] else None
    gw = dev(g.load_f32(m["gate_vec"].name).reshape(-1)) if (m["gate_vec"] is not None and shared) else None
    return MoeLayer(router, gate, up, down, m["expert_type"], int(K), shared=shared,
                    shared_type=m["shared_type"] if shared else None, sh_gate_w=gw, max_ntok=max_ntok)
