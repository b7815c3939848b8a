"""The C-ABI library loads and exports every symbol include/*.h declares, and
rejects bad descriptors with a status before any launch (CPU-only: these
calls return before touching the GPU)."""
import ctypes as C
import glob
import os
import re

import pytest

import npu_amd
from npu_amd import _lib
from npu_amd.memref import BF16, F32, I8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header):
    names = set()
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, re.M):
        if m.group(1) not in ("if", "return", "sizeof"):
            names.add(m.group(1))
    return names


def test_headers_cover_every_library():
    assert sorted(os.path.basename(h) for h in glob.glob(os.path.join(ROOT, "include", "*.h"))) \
        == ["npu_amd.h", "npu_cost.h"]


def test_header_declares_entry_points():
    names = declared_functions("npu_amd.h")
    assert {"fused_matmul_bias_act", "fused_conv2d_nhwc_bias_act", "npu_last_error"} <= names


def test_library_exports_every_declared_symbol():
    lib = npu_amd.lib()
    missing = [n for n in sorted(declared_functions("npu_amd.h")) if not hasattr(lib, n)]
    assert not missing, f"declared in npu_amd.h but not exported: {missing}"
    assert set(_lib.SIGNATURES) == declared_functions("npu_amd.h")


def test_host_library_exports_every_declared_symbol():
    from npu_amd import host
    h = host.lib()
    missing = [n for n in sorted(declared_functions("npu_cost.h")) if not hasattr(h, n)]
    assert not missing, f"declared in npu_cost.h but not exported: {missing}"
    assert set(host.SIGNATURES) == declared_functions("npu_cost.h")


def test_version_and_status_strings():
    lib = npu_amd.lib()
    assert b"gfx950" in lib.npu_version()
    assert lib.npu_status_string(0) == b"ok"
    assert lib.npu_status_string(2) == b"unsupported"


def _mr(shape, dtype=F32, ptr=0x10000, strides=None):
    m = _lib.NpuMemref()
    m.allocated = m.aligned = ptr
    m.offset = 0
    st = strides or [int(__import__("numpy").prod(shape[i + 1:])) for i in range(len(shape))]
    for i, (s, t) in enumerate(zip(shape, st)):
        m.sizes[i], m.strides[i] = s, t
    m.rank, m.dtype = len(shape), dtype
    return m


def _err():
    return npu_amd.lib().npu_last_error().decode()


def test_matmul_rejects_bad_descriptors():
    lib = npu_amd.lib()
    A, B, b, o = _mr([8, 16]), _mr([16, 4]), _mr([4]), _mr([8, 4])
    call = lambda *a: lib.fused_matmul_bias_act(*[C.byref(x) if x is not None else None for x in a[:4]], a[4], None)
    assert call(None, B, b, o, 1) == 1 and "A" in _err()
    assert call(A, _mr([15, 4]), b, o, 1) == 1 and "expected K" in _err()
    assert call(A, B, b, _mr([8, 5]), 1) == 1 and "out" in _err()
    assert call(A, B, _mr([5]), o, 1) == 1 and "bias" in _err()
    assert call(A, _mr([16, 4], BF16), b, o, 1) == 1 and "dtype" in _err()
    assert call(A, B, b, o, 7) == 1 and "act" in _err()
    assert call(_mr([8, 6]), _mr([6, 4]), b, o, 1) == 2 and "multiple of 4" in _err()
    assert call(A, _mr([16, 4], strides=[1, 16]), b, o, 1) == 2 and "contiguous" in _err()
    assert call(_mr([8, 16], ptr=0x10004), B, b, o, 1) == 2 and "aligned" in _err()


def test_irb_channel_limits():
    """fused_irb_f32 takes C % 4 == 0 in [4, 320] and E % 16 == 0 (the tuned
    (C, E) pairs and the streaming kernel); other counts are refused by name
    before any launch."""
    lib = npu_amd.lib()

    def call(ch, e):
        x, o = _mr([1, 4, 4, ch]), _mr([1, 4, 4, ch])
        we, wdw, wp = _mr([e, ch]), _mr([3, 3, e]), _mr([ch, e])
        return lib.fused_irb_f32(*[C.byref(m) for m in (x, we, wdw, wp, o)], None)

    for ch, e in ((324, 1280), (26, 144), (24, 100), (40, 24)):
        assert call(ch, e) == 2 and "multiple of 4 in [4, 320]" in _err(), (ch, e, _err())


def test_qbottleneck_channel_limits():
    """fused_qbottleneck_i8 takes C % 64 == 0 up to 2048 and M1 % 64 == 0 up
    to 512; other counts are refused by name before any launch."""
    from npu_amd.memref import I32
    lib = npu_amd.lib()

    def call(ch, m1):
        ms = [_mr([1, 4, 4, ch], I8), _mr([m1, ch], I8), _mr([m1, 3, 3, m1], I8), _mr([ch, m1], I8)]
        ms += [_mr([m1], I32), _mr([m1], I32), _mr([m1], I32), _mr([m1], I32), _mr([ch], I32),
               _mr([ch], I32), _mr([1, 4, 4, ch], I8)]
        return lib.fused_qbottleneck_i8(*[C.byref(m) for m in ms], None)

    for ch, m1 in ((96, 64), (4096, 64), (256, 576), (256, 96)):
        assert call(ch, m1) == 2 and "multiple of 64" in _err(), (ch, m1, _err())


def test_conv_rejects_bad_descriptors():
    lib = npu_amd.lib()
    x, w, b, o = _mr([1, 8, 8, 16]), _mr([16, 3, 3, 16]), _mr([16]), _mr([1, 8, 8, 16])
    call = lambda x_, w_, b_, o_, pad=1, act=1: lib.fused_conv2d_nhwc_bias_act(
        C.byref(x_), C.byref(w_), C.byref(b_), C.byref(o_), pad, act, None)
    assert call(x, w, b, _mr([1, 7, 8, 16])) == 1 and "out" in _err()
    assert call(x, _mr([16, 3, 3, 8]), b, o) == 1 and "channels" in _err()
    assert call(_mr([1, 8, 8, 16], I8), w, b, o) == 2 and "f32 or bf16" in _err()
    assert call(_mr([1, 8, 8, 22]), _mr([16, 3, 3, 22]), b, o) == 2 and "multiple of 4" in _err()
    assert call(x, w, b, o, pad=-1) == 1 and "negative" in _err()
    xb = _mr([1, 8, 8, 12], BF16)
    assert call(xb, _mr([16, 3, 3, 12], BF16), b, _mr([1, 8, 8, 16], BF16)) == 2 and "8" in _err()
    # the residual variant checks the residual against the output
    res = lambda r_: lib.fused_conv2d_nhwc_bias_res_act(
        C.byref(x), C.byref(w), C.byref(b), C.byref(r_), C.byref(o), 1, 1, None)
    assert res(_mr([1, 8, 7, 16])) == 1 and "res" in _err()
    assert res(_mr([1, 8, 8, 16], BF16)) == 1 and "res" in _err()


def test_python_mirror_raises_with_library_message():
    torch = pytest.importorskip("torch")
    A = torch.zeros(4, 6)  # host tensors: validation fails before any launch
    with pytest.raises(npu_amd.NpuError, match="multiple of 4"):
        npu_amd.fused_matmul_bias_act(A, torch.zeros(6, 4), None, torch.zeros(4, 4), "relu", 0)


def test_qbottleneck_rejects_bad_descriptors():
    lib = npu_amd.lib()
    from npu_amd.memref import I32
    x, w1, w2, w3 = _mr([1, 8, 8, 256], I8), _mr([64, 256], I8), _mr([64, 3, 3, 64], I8), _mr([256, 64], I8)
    q = [_mr([64], I32), _mr([64], I32), _mr([64], I32), _mr([64], I32), _mr([256], I32), _mr([256], I32)]
    o = _mr([1, 8, 8, 256], I8)

    def call(*a):
        return lib.fused_qbottleneck_i8(*[C.byref(m) for m in a], None)

    assert call(x, w1, w2, w3, *q, _mr([1, 8, 8, 128], I8)) == 1 and "out" in _err()
    assert call(x, _mr([64, 128], I8), w2, w3, *q, o) == 1 and "w1" in _err()
    assert call(x, w1, _mr([64, 3, 3, 32], I8), w3, *q, o) == 1 and "w2" in _err()
    assert call(x, w1, w2, w3, *q[:4], _mr([64], I32), q[5], o) == 1 and "m3" in _err()
    assert call(x, w1, w2, w3, _mr([64], F32), *q[1:], o) == 1 and "dtype" in _err()
    xx, ww1 = _mr([1, 8, 8, 160], I8), _mr([64, 160], I8)
    assert call(xx, ww1, w2, _mr([160, 64], I8), *q[:4], _mr([160], I32), _mr([160], I32),
                _mr([1, 8, 8, 160], I8)) == 2 and "multiple of 64" in _err()


C_TEST = os.path.join(ROOT, "tests", "c", "group_launch_test")


def test_compiled_c_caller_gets_rejections_before_launch():
    """A C program calls npu_group_launch with wrong counts, shapes, ranks,
    fill values and chain names; each is refused with a status and message."""
    import subprocess
    assert os.path.exists(C_TEST), "build tests/c first (__graft_entry__.build())"
    r = subprocess.run([C_TEST, "validate"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr


def _arg2(shape, ptr=0x10000):
    from npu_amd import groups
    d = _lib.strided_memref_type(len(shape))()
    d.allocated = d.aligned = ptr
    st = 1
    for i in range(len(shape) - 1, -1, -1):
        d.sizes[i], d.strides[i] = shape[i], st
        st *= shape[i]
    a = _lib.NpuArg()
    a.rank, a.descriptor, a.dtype, a.kind = len(shape), C.addressof(d), F32, 0
    a._keep = d
    return a


def test_group_launch_reads_strided_memref_layouts():
    """The descriptor is MLIR's StridedMemRefType layout for each rank: a conv
    group's 4-D and 1-D arguments are read from their own layouts (the
    rejection names the right shapes)."""
    lib = npu_amd.lib()
    sc = _lib.NpuArg()
    sc.kind, sc.scalar = 1, 0.0
    at = _lib.NpuGroupAttrs()
    at.act[0], at.pad = 1, 1
    ins = [sc, _arg2([2, 8, 8, 32]), _arg2([2, 8, 8, 16]), _arg2([32, 3, 3, 16]), _arg2([31]),
           _arg2([2, 8, 8, 32])]
    outs = [_arg2([2, 8, 8, 32])]
    ia, oa = (_lib.NpuArg * 6)(*ins), (_lib.NpuArg * 1)(*outs)
    st = lib.npu_group_launch(b"fused_fill_linalg_conv_2d_nhwc_fhwc_generic_0", C.byref(at),
                              ia, 6, oa, 1, None)
    assert st == 1 and "bias: size 31, expected F = 32" in _err()
    # one dimension off in the accumulator
    ins[1] = _arg2([2, 8, 7, 32])
    ia = (_lib.NpuArg * 6)(*ins)
    st = lib.npu_group_launch(b"fused_fill_linalg_conv_2d_nhwc_fhwc_generic_0", C.byref(at),
                              ia, 6, oa, 1, None)
    assert st == 1 and "accumulator" in _err()


def test_zero_sized_dimensions_are_rejected_before_launch():
    """A memref with a zero-sized dimension is refused with INVALID_ARG (the
    reference's groups have static, nonzero shapes), whichever operand it
    is, with no launch."""
    lib = npu_amd.lib()
    call = lambda *a: lib.fused_matmul_bias_act(*[C.byref(x) for x in a[:4]], a[4], None)
    A, B, b, o = _mr([8, 16]), _mr([16, 4]), _mr([4]), _mr([8, 4])
    for args in ((_mr([0, 16]), B, b, _mr([0, 4])), (A, _mr([16, 0]), _mr([0]), _mr([8, 0])),
                 (_mr([8, 0]), _mr([0, 4]), b, o)):
        assert call(*args, 1) == 1
        assert "must be positive" in _err()
