"""GGUF ingestion (chimere_amd/gguf.py): the reader against hand-packed bytes
of the format (cs/src/gguf_loader.rs:298-696), its error cases, the writer by
round trip, and the mapping of one MoE layer's tensors onto the fused layer
(cs/src/qwen35_model/compute_graph.rs:988-1000, 1395-1440); on the GPU a
layer built from a GGUF file is bit-exact against the oracle."""
import struct

import numpy as np
import pytest

import oracle as O
from chimere_amd import gguf as GG


def s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def handmade(tmp_path, version=3, magic=0x46554747, extra_kv=b"", n_kv_extra=0, qtype=8, trunc=0, align_kv=None):
    """Two tensors: 'a' F32 [4] and 'b' Q8_0 dims [32, 2] (2 rows of one block)."""
    kv = s("general.architecture") + struct.pack("<I", 8) + s("qwen35moe")
    kv += s("qwen35moe.expert_used_count") + struct.pack("<II", 4, 8)
    kv += s("tokenizer.scores") + struct.pack("<IIQ", 9, 6, 2) + struct.pack("<ff", 0.5, -1.0)
    nkv = 3 + n_kv_extra
    al = 32
    if align_kv is not None:
        kv += s("general.alignment") + struct.pack("<II", 4, align_kv)
        nkv += 1
        al = align_kv
    kv += extra_kv
    ti = s("a") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 0)
    off_b = 32 if al <= 32 else al
    ti += s("b") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", qtype, off_b)
    head = struct.pack("<IIQQ", magic, version, 2, nkv) + kv + ti
    head += b"\0" * ((-len(head)) % al)
    a = np.array([1.0, -2.0, 3.5, 0.25], np.float32).tobytes()
    blk = struct.pack("<e", 0.5) + bytes(range(32))
    data = a + b"\0" * (off_b - len(a)) + blk + blk[::-1]
    p = tmp_path / "t.gguf"
    p.write_bytes((head + data)[:len(head + data) - trunc])
    return p, len(head)


def test_read_handmade(tmp_path):
    p, hl = handmade(tmp_path)
    g = GG.GgufFile(p)
    assert g.version == 3 and g.n_tensors == 2 and g.n_kv == 3 and g.alignment == 32
    assert g.data_section_offset == hl and hl % 32 == 0
    assert g.get_metadata("general.architecture") == "qwen35moe"
    assert g.get_metadata("qwen35moe.expert_used_count") == 8
    assert g.get_metadata("tokenizer.scores") == [0.5, -1.0]
    assert g.tensor_names() == ["a", "b"] and g.tensor_ggml_type("b") == GG.Q8_0
    b = g.get_tensor_info("b")
    assert b.dims == (32, 2) and b.n_elements == 64 and b.nbytes == 68
    assert (g.load_f32("a") == np.array([1.0, -2.0, 3.5, 0.25], np.float32)).all()
    raw = g.tensor_data("b")
    assert raw[:2].view(np.float16)[0] == 0.5 and (raw[2:34] == np.arange(32)).all()
    assert g.get_tensor_info("missing") is None
    with pytest.raises(GG.GgufError, match="not found"):
        g.tensor_data("missing")


def test_custom_alignment(tmp_path):
    p, hl = handmade(tmp_path, align_kv=64)
    g = GG.GgufFile(p)
    assert g.alignment == 64 and g.data_section_offset % 64 == 0
    assert g.tensor_data("b")[:2].view(np.float16)[0] == 0.5


@pytest.mark.parametrize("kw,msg", [
    (dict(magic=0x46554748), "Invalid GGUF magic"),
    (dict(version=1), "Unsupported GGUF version: 1"),
    (dict(version=4), "Unsupported GGUF version: 4"),
    (dict(qtype=5), "Unknown GGML type 5 for tensor 'b'"),
    (dict(extra_kv=s("k") + struct.pack("<I", 13), n_kv_extra=1), "Unknown GGUF value type: 13"),
    (dict(extra_kv=s("k") + struct.pack("<IQ", 8, 10**6), n_kv_extra=1), "String extends beyond file"),
    (dict(trunc=10), "data extends beyond file"),
])
def test_errors(tmp_path, kw, msg):
    trunc = kw.pop("trunc", 0)
    p, _ = handmade(tmp_path, trunc=trunc, **kw)
    with pytest.raises(GG.GgufError, match=msg):
        g = GG.GgufFile(p)
        g.tensor_data("b")


def test_block_info_matches_reference_table():
    # cs/src/gguf_loader.rs:161-194, the types of this path
    assert GG.BLOCK_INFO[GG.Q4_0] == (32, 18) and GG.BLOCK_INFO[GG.Q8_0] == (32, 34)
    assert GG.BLOCK_INFO[GG.IQ3_S] == (256, 110) and GG.BLOCK_INFO[GG.Q5_K] == (256, 176)
    assert GG.BLOCK_INFO[GG.Q4_K] == (256, 144) and GG.BLOCK_INFO[GG.Q6_K] == (256, 210)
    assert GG.tensor_bytes(GG.IQ3_S, 256 * 512 * 2048) == 256 * 512 * 2048 // 256 * 110
    for t in (GG.Q4_0, GG.Q8_0, GG.IQ3_S):
        assert GG.tensor_bytes(t, 2048) == O.row_bytes(t, 2048)


def write_moe_gguf(path, H=512, F=256, E=8, K=4, et=O.Q4_0, st=O.Q8_0, seed=0, layer=3):
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    q = lambda t, r, c, n: O.quantize(t, (rng.standard_normal((n * r, c)) * 0.02).astype(np.float32))  # noqa: E731
    gate, up, down = q(et, F, H, E), q(et, F, H, E), q(et, H, F, E)
    sh = (q(st, F, H, 1), q(st, F, H, 1), q(st, H, F, 1))
    gw = (rng.standard_normal(H) * 0.02).astype(np.float32)
    b = f"blk.{layer}."
    tensors = [(b + "ffn_gate_inp.weight", (H, E), GG.F32, router.tobytes()),
               (b + "ffn_gate_exps.weight", (H, F, E), et, gate.tobytes()),
               (b + "ffn_up_exps.weight", (H, F, E), et, up.tobytes()),
               (b + "ffn_down_exps.weight", (F, H, E), et, down.tobytes()),
               (b + "ffn_gate_shexp.weight", (H, F), st, sh[0].tobytes()),
               (b + "ffn_up_shexp.weight", (H, F), st, sh[1].tobytes()),
               (b + "ffn_down_shexp.weight", (F, H), st, sh[2].tobytes()),
               (b + "ffn_gate_inp_shexp.weight", (H,), GG.F32, gw.tobytes())]
    md = {"general.architecture": (GG.STRING, "qwen35moe"), "qwen35moe.expert_used_count": (GG.UINT32, K),
          "qwen35moe.expert_count": (GG.UINT32, E)}
    GG.write_gguf(path, md, tensors)
    return dict(router=router, gate=gate.reshape(E, -1), up=up.reshape(E, -1), down=down.reshape(E, -1),
                sh=tuple(m.reshape(-1) for m in sh), gw=gw, H=H, F=F, E=E, K=K, et=et, st=st)


def test_writer_round_trip_and_moe_mapping(tmp_path):
    ref = write_moe_gguf(tmp_path / "m.gguf")
    g = GG.GgufFile(tmp_path / "m.gguf")
    assert g.data_section_offset % 32 == 0
    assert all(t.data_offset % 32 == 0 for t in g.tensors)
    m = GG.moe_tensors(g, 3)
    assert (m["H"], m["F"], m["E"], m["K"]) == (ref["H"], ref["F"], ref["E"], ref["K"])
    assert m["expert_type"] == ref["et"] and m["shared_type"] == ref["st"]
    assert (g.load_f32("blk.3.ffn_gate_inp.weight") == ref["router"]).all()
    assert (g.tensor_data("blk.3.ffn_down_exps.weight").reshape(ref["E"], -1) == ref["down"]).all()
    assert (g.tensor_data("blk.3.ffn_up_shexp.weight") == ref["sh"][1]).all()
    assert (g.load_f32("blk.3.ffn_gate_inp_shexp.weight") == ref["gw"]).all()
    with pytest.raises(GG.GgufError, match="not found"):
        GG.moe_tensors(g, 4)


def test_moe_mapping_rejects_mismatched_dims(tmp_path):
    H, F, E = 512, 256, 4
    z = lambda t, n: bytes(GG.tensor_bytes(t, n))   # noqa: E731
    tensors = [("blk.0.ffn_gate_inp.weight", (H, E), GG.F32, z(GG.F32, H * E)),
               ("blk.0.ffn_gate_exps.weight", (H, F, E), GG.Q4_0, z(GG.Q4_0, H * F * E)),
               ("blk.0.ffn_up_exps.weight", (H, F, E), GG.Q4_0, z(GG.Q4_0, H * F * E)),
               ("blk.0.ffn_down_exps.weight", (H, F, E), GG.Q4_0, z(GG.Q4_0, H * F * E))]   # down not [F, H, E]
    GG.write_gguf(tmp_path / "bad.gguf", {}, tensors)
    with pytest.raises(GG.GgufError, match="do not match"):
        GG.moe_tensors(GG.GgufFile(tmp_path / "bad.gguf"), 0)


@pytest.mark.gpu
def test_moe_layer_from_gguf_bit_exact(tmp_path, dev):
    import torch
    ref = write_moe_gguf(tmp_path / "m.gguf", H=1024, F=256, E=16, K=4, seed=3)
    g = GG.GgufFile(tmp_path / "m.gguf")
    layer = GG.moe_layer_from_gguf(g, 3, dev)
    x = torch.randn(2, 1024, generator=torch.Generator(device=dev).manual_seed(1), device=dev)
    out = layer.forward(x)
    torch.cuda.synchronize()
    oo, _, _ = O.moe(x.cpu().numpy(), ref["router"], ref["gate"], ref["up"], ref["down"], ref["et"], ref["K"],
                     sh=ref["sh"], sh_type=ref["st"], sh_gate_w=ref["gw"])
    assert (out.cpu().numpy().view(np.uint32) == oo.view(np.uint32)).all()
