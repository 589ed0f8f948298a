"""CPU-side checks of the C-ABI library and the host layer (no GPU compute calls)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "flint_amd.h")).read()
    return sorted(set(re.findall(r"^int\s+(fl_\w+)\s*\(", src, flags=re.M)))


def test_header_matches_binding():
    from flint_amd import _lib
    assert _declared_symbols() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    from flint_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run python -m flint_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert _lib.load().fl_version() >= 1


def test_argument_errors_without_gpu():
    """Entry points reject bad arguments before touching the device."""
    from flint_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    lib = _lib.load()
    assert lib.fl_quantize_int4(None, None, None, 16, 128, None) == -1
    assert lib.fl_dequant_int4(None, None, None, 16, 128, None) == -1
    assert lib.fl_dequant_int4_mx(None, None, None, 16, 128, None) == -1
    p = ctypes.c_void_p(16)
    assert lib.fl_gemv_int4(p, p, p, p, 16, 100, None) == -1       # K not a multiple of 128
    assert lib.fl_gemv_int4(p, p, p, p, 0, 128, None) == -1
    desc = _lib.ModelDesc(1, 500, 8, 2, 1024, 1024, 1e-5, 1.0, 0.125, 1.0, 1.0)  # dim % 128 != 0
    st = ctypes.c_void_p()
    assert lib.fl_state_create(ctypes.byref(desc), 64, p, p, ctypes.byref(st)) == -1
    desc = _lib.ModelDesc(1, 512, 8, 3, 1024, 1024, 1e-5, 1.0, 0.125, 1.0, 1.0)  # 8 % 3 != 0
    assert lib.fl_state_create(ctypes.byref(desc), 64, p, p, ctypes.byref(st)) == -1
    assert lib.fl_state_create(ctypes.byref(desc), 64, None, p, ctypes.byref(st)) == -1
    assert lib.fl_decode_step(None, None, None, 0, None, None, None, None) == -1
    # hand-off probe modes: kind 3 takes a depth of 1..3 and a word count divisible by 4
    g = ctypes.c_int32()
    assert lib.fl_probe_handoff(5, 64, 10, p, ctypes.byref(g), None) == -1            # no kind 5
    assert lib.fl_probe_handoff(4 | 1 << 8, 64, 10, p, ctypes.byref(g), None) == -1   # kind 4: no knobs
    assert lib.fl_probe_handoff(4, 66, 10, p, ctypes.byref(g), None) == -1            # kind 4: 66 % 4
    assert lib.fl_probe_handoff(3, 64, 10, p, ctypes.byref(g), None) == -1            # depth 0
    assert lib.fl_probe_handoff(3 | 4 << 8, 64, 10, p, ctypes.byref(g), None) == -1   # depth 4
    assert lib.fl_probe_handoff(3 | 1 << 8, 66, 10, p, ctypes.byref(g), None) == -1   # 66 % 4
    assert lib.fl_probe_handoff(1 | 1 << 8, 64, 10, p, ctypes.byref(g), None) == -1   # extra bits
    assert lib.fl_probe_dequant(5, 10, p, ctypes.byref(g), None) == -1                 # no mode 5
    assert lib.fl_probe_dequant(0, 0, p, ctypes.byref(g), None) == -1                 # iters >= 1


def test_storage_permutations():
    from flint_amd.model import gu_storage_rows, qkv_storage_perm
    from flint_amd.synth import ModelArgs
    a = ModelArgs.from_name("tiny")
    perm = qkv_storage_perm(a)
    assert sorted(perm.tolist()) == list(range(a.qkv_dim))
    # packed rows 2i / 2i+1 of head h are model rows h*64+i / h*64+i+32
    for h in range(a.n_head + 2 * a.n_local_heads):
        for i in range(32):
            assert perm[h * 64 + 2 * i] == h * 64 + i
            assert perm[h * 64 + 2 * i + 1] == h * 64 + i + 32
    w1 = torch.arange(6).view(3, 2)
    w3 = 10 + torch.arange(6).view(3, 2)
    gu = gu_storage_rows(w1, w3)
    assert torch.equal(gu[0::2], w1) and torch.equal(gu[1::2], w3)


def test_unpack_helpers_roundtrip():
    from flint_amd.quantize import pack_q, unpack_q, unpack_sz
    vals = torch.randint(0, 16, (4, 64), dtype=torch.int32)
    words = pack_q(vals)
    assert torch.equal(unpack_q(words), vals)
    # element 2i of a word at bits 4i, element 2i+1 at bits 16+4i
    one = torch.zeros(1, 8, dtype=torch.int32)
    one[0, 3] = 5
    assert int(pack_q(one)[0, 0]) == 5 << 20
    s = torch.randn(3, 2).to(torch.bfloat16)
    z = torch.randn(3, 2).to(torch.bfloat16)
    packed = (s.view(torch.int16).to(torch.int32) & 0xFFFF) | (z.view(torch.int16).to(torch.int32) << 16)
    s2, z2 = unpack_sz(packed)
    assert torch.equal(s2, s) and torch.equal(z2, z)


def test_bench_rejects_multi_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr


def test_torch_extension_loads():
    """The torch-extension binding (flint_amd/_torch_ops*.so, built by flint_amd.build) imports on
    the CPU and exposes the reference's op forms over torch tensors; argument checks run before
    any device call."""
    from flint_amd import build
    if not os.path.exists(build.torch_ext_path()):
        pytest.skip("torch extension not built (run python -m flint_amd.build)")
    import flint_amd._torch_ops as ops
    assert ops.version() >= 1
    for name in ("decode_hidden", "decode_step", "verify", "check"):
        assert hasattr(ops.Engine, name)
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    q = torch.zeros(8, 32, dtype=torch.int32)
    sz = torch.zeros(8, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="device tensor"):
        ops.int4_linear(x, q, sz, 0)
