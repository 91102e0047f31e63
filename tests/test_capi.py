"""C-ABI checks that need no GPU: the library loads, exports every function
include/chimere_hip.h declares, the binding covers them, and argument
validation rejects bad calls before any launch (the reference's ABI has no
error channel; this one records CHIMERE_ERR_* per host thread)."""
import ctypes as C
import os
import re

import pytest

from chimere_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    txt = open(os.path.join(ROOT, "include", "chimere_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(chimere_[a-z0-9_]+)\s*\(", txt)))


def test_header_symbols_exported_and_bound():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), f"{n} not exported by libchimere_hip.so"
    bound = {s[0] for s in _lib.SIGNATURES}
    assert set(names) == bound


def test_size_helpers():
    L = _lib.lib()
    assert L.chimere_q8_1_block_bytes() == 36
    assert L.chimere_q8_1_block_elems() == 32
    assert L.chimere_matrix_row_padding() == 512


def _err():
    L = _lib.lib()
    msg = L.chimere_hip_get_last_error_string().decode()
    return L.chimere_hip_get_last_error(), msg


def test_validation_rejects_without_launch():
    L = _lib.lib()
    assert _err()[0] == 0
    L.chimere_mmvq_q8_0(None, None, None, 2048, 16, 64, None)
    code, msg = _err()
    assert code == 1 and "null" in msg
    assert _err()[0] == 0                                  # reading clears it
    fake = C.c_void_p(0x1000)
    L.chimere_mmvq_q4_0(fake, fake, fake, 2000, 16, 64, None)    # ncols % 32
    assert _err()[0] == 1
    L.chimere_mmvq_iq3s(fake, fake, fake, 2048 + 32, 16, 66, None)  # ncols % 256
    assert _err()[0] == 1
    L.chimere_mmvq_q8_0(fake, fake, fake, 2048, 16, 10, None)     # nrows_y_padded too small
    assert _err()[0] == 1
    L.chimere_mmvq_multi(8, fake, fake, fake, 2048, 16, 64, 9, None)  # ntok > 8
    assert _err()[0] == 1
    L.chimere_mmvq_q8_0_batched(fake, fake, fake, None, 2048, 16, 64, 1 << 20, 0, 8, None)  # ids NULL
    assert _err()[0] == 1
    L.chimere_quantize_q8_1(fake, fake, 100, 64, None)           # padded < ncols
    assert _err()[0] == 1
    L.chimere_quantize_weights(5, fake, fake, 64, None)          # unknown type
    assert _err()[0] == 1
    L.chimere_topk_softmax(fake, fake, fake, 2048, 8, 1, None)   # E > 1024
    assert _err()[0] == 1


def _layer(**kw):
    c = _lib.MoeLayerC()
    c.hidden, c.ffn, c.n_experts, c.top_k = 2048, 512, 256, 8
    c.expert_type, c.shared_type = 2, 2
    for f in ("router_w", "gate_exps", "up_exps", "down_exps", "sh_gate", "sh_up", "sh_down"):
        setattr(c, f, 0x1000)
    c.gate_stride = c.up_stride = c.down_stride = 589824
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_moe_workspace_and_validation():
    L = _lib.lib()
    c = _layer()
    ws1 = L.chimere_moe_workspace_size(C.byref(c), 1)
    ws8 = L.chimere_moe_workspace_size(C.byref(c), 8)
    assert 0 < ws1 < ws8 < (1 << 24)
    assert L.chimere_moe_workspace_size(C.byref(c), 9) == 0
    x = C.c_void_p(0x1000)
    ws = C.c_void_p(0x100000)
    L.chimere_moe_ffn_decode(C.byref(c), x, x, 1, None, None, ws, ws1 - 1, None)
    assert _err()[0] == 3                                   # workspace too small
    for bad in (dict(top_k=17), dict(n_experts=2048), dict(hidden=2000), dict(expert_type=7),
                dict(gate_stride=100), dict(sh_up=None)):
        c = _layer(**bad)
        L.chimere_moe_ffn_decode(C.byref(c), x, x, 1, None, None, ws, 1 << 30, None)
        assert _err()[0] == 1, bad
    c = _layer()
    L.chimere_moe_ffn_decode(C.byref(c), x, x, 0, None, None, ws, 1 << 30, None)   # ntok 0
    assert _err()[0] == 1
