"""C-ABI checks that need no GPU: libtq.so loads, exports every entry point
include/tq.h declares, and rejects bad arguments on the host before any launch."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from turboquant.runtime import _lib
from turboquant.runtime import kernels as K
from turboquant.runtime.params import layer_codecs

HEADER = Path(__file__).resolve().parent.parent / "include" / "tq.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tq_\w+)\s*\(", text, flags=re.M))


def test_header_and_binding_agree():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.tq_abi_version() == _lib.ABI_VERSION == 1


def test_status_strings():
    lib = _lib.load()
    assert lib.tq_status_string(0) == b"ok"
    for s in (1, 2, 3, 4):
        assert lib.tq_status_string(s) not in (b"ok", b"unknown status")
    assert lib.tq_status_string(99) == b"unknown status"


FAKE = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: validation fails first


def test_quantize_rejects_bad_arguments_on_host():
    lib = _lib.load()
    # null input
    assert lib.tq_quantize_mse(None, 1, 1, 1, 128, 128, 128, 128, 4, FAKE, FAKE, FAKE, FAKE, 1, 0, None) == 1
    # head_dim 64 is not built
    assert lib.tq_quantize_mse(FAKE, 1, 1, 1, 64, 64, 64, 64, 4, FAKE, FAKE, FAKE, FAKE, 1, 0, None) == 2
    # writes past the capacity
    assert lib.tq_quantize_mse(FAKE, 1, 1, 4, 128, 512, 512, 128, 4, FAKE, FAKE, FAKE, FAKE, 4, 1, None) == 1
    # bad bit widths
    assert lib.tq_quantize_mse(FAKE, 1, 1, 1, 128, 128, 128, 128, 5, FAKE, FAKE, FAKE, FAKE, 1, 0, None) == 1
    assert lib.tq_quantize_prod(FAKE, 1, 1, 1, 128, 128, 128, 128, 4, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                FAKE, 1, 0, None) == 1
    # misaligned strides
    assert lib.tq_quantize_mse(FAKE, 1, 1, 1, 128, 130, 130, 130, 4, FAKE, FAKE, FAKE, FAKE, 1, 0, None) == 2


def test_attention_rejects_bad_arguments_on_host():
    lib = _lib.load()
    args = dict(q=FAKE, batch=1, q_heads=8, kv_heads=2, dim=128, starts=None, lens=None, n=16, cap=16, kc=FAKE,
                kn=FAKE, ks=FAKE, kr=FAKE, vc=FAKE, vn=FAKE, kb=3, vb=4, qjl=1, rk=FAKE, ck=FAKE, s=FAKE, rv=FAKE,
                cv=FAKE, scale=ctypes.c_float(0.0), of=FAKE, ob=FAKE, lse=None, ws=FAKE, wsb=1 << 30, stream=None)

    def call(**kw):
        a = dict(args, **kw)
        return lib.tq_decode_attention(*a.values())

    assert call(q_heads=9) == 1          # Hq not a multiple of Hkv
    assert call(q_heads=18) == 2         # GQA group 9 > 8
    assert call(dim=64) == 2
    assert call(kb=4, vb=4) == 2         # Q_prod needs key_bits = value_bits - 1
    assert call(qjl=0, kb=3, vb=4) == 2  # Q_mse needs equal widths
    assert call(ws=None) == 3
    assert call(wsb=16) == 3
    assert call(cap=8) == 1              # n_tokens > cap
    assert call(ks=None) == 1            # QJL without signs
    assert call(of=None, ob=None) == 1


def test_workspace_size_is_host_arithmetic():
    lib = _lib.load()
    small = lib.tq_decode_attention_workspace_bytes(1, 8, 2, 128, 100)
    big = lib.tq_decode_attention_workspace_bytes(8, 32, 8, 128, 32768)
    assert 0 < small <= big
    assert lib.tq_decode_attention_workspace_bytes(1, 8, 2, 64, 100) == 0


def test_wrappers_refuse_cpu_tensors():
    """No CPU fallback: the product path raises instead of computing on the host."""
    lc = layer_codecs(128, 4, 0, True, "cpu")
    x = torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16)
    codes = torch.zeros(1, 1, 4, 64, dtype=torch.uint8)
    norms = torch.zeros(1, 1, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        K.quantize_mse(x, lc.value, codes, norms)
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        K.decode_attention(q, k_codes=codes, k_norms=norms, v_codes=codes, v_norms=norms, n_tokens=4,
                           key=lc.key, value=lc.value)


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libtq.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="not built"):
        _lib.load()
