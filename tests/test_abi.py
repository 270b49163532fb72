"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/muonadamw_amd.h, and rejects invalid arguments on the host
(negative status codes) before making any HIP call.  Device pointers here are
fake addresses: validation never dereferences them."""

import ctypes
import re
from pathlib import Path

import pytest

from triton_muon_adamw import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "muonadamw_amd.h"

OK, NULL, COUNT, NUMEL, SHAPE, ALIGN, WS, HYPER, TABLE, ALIAS, SCRATCH = 0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mamw_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "mamw_muon_step" in names and "mamw_adamw_mt_step" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _lib._PROTOTYPES, f"{name} has no ctypes prototype"


def test_version_and_strerror():
    lib = _lib.load()
    assert lib.mamw_abi_version() == 5
    for code in (OK, NULL, COUNT, NUMEL, SHAPE, ALIGN, WS, HYPER, TABLE, ALIAS, SCRATCH):
        msg = lib.mamw_strerror(code).decode()
        assert msg and msg != "unknown status"
    assert lib.mamw_strerror(-1234).decode() == "unknown status"
    with pytest.raises(ValueError, match="NULL"):
        _lib.check(NULL, "x")


# ---- AdamW table ---------------------------------------------------------------

def _t(base, numel, stride=1 << 30):
    return _lib.AdamWTensor(base, base + stride, base + 2 * stride, base + 3 * stride, numel)


def _pack(tensors):
    lib = _lib.load()
    n = len(tensors)
    arr = (_lib.AdamWTensor * max(n, 1))(*tensors)
    nbytes = ctypes.c_size_t()
    assert lib.mamw_adamw_table_bytes(n, ctypes.byref(nbytes)) == OK
    assert nbytes.value == 64 * (n + 1)  # + the record the device-counter step writes
    buf = (ctypes.c_uint8 * max(nbytes.value, 1))()
    blocks = ctypes.c_int64(-1)
    st = lib.mamw_adamw_table_pack(arr, n, buf, nbytes.value, ctypes.byref(blocks))
    return st, bytes(buf), blocks.value


def test_adamw_pack_blocks_and_records():
    st, buf, blocks = _pack([_t(1 << 40, 4096), _t(2 << 40, 1), _t(3 << 40, 0), _t(4 << 40, 10000)])
    assert st == OK
    assert blocks == 4 + 1 + 0 + 10  # 1024-element chunks
    import struct

    begins = [struct.unpack_from("<q", buf, 64 * i + 40)[0] for i in range(4)]
    assert begins == [0, 4, 5, 5]
    vec_ok = [struct.unpack_from("<i", buf, 64 * i + 48)[0] for i in range(4)]
    assert vec_ok == [1, 1, 1, 1]
    st, buf, _ = _pack([_t((1 << 40) + 4, 100)])  # 4-byte aligned, not 16
    assert st == OK and struct.unpack_from("<i", buf, 48)[0] == 0


def _pack_ex(entries):
    lib = _lib.load()
    n = len(entries)
    arr = (_lib.AdamWTensorEx * max(n, 1))(*entries)
    buf = (ctypes.c_uint8 * (64 * (n + 1)))()
    blocks = ctypes.c_int64(-1)
    st = lib.mamw_adamw_table_pack_ex(arr, n, buf, 64 * (n + 1), ctypes.byref(blocks))
    return st, bytes(buf), blocks.value


def _tx(base, numel, flags, pstep=1 << 30):
    return _lib.AdamWTensorEx(base, base + pstep, base + 2 * pstep, base + 3 * pstep, numel, flags, 0)


def test_adamw_pack_ex_flags_and_alignment():
    import struct

    BP, BG = _lib.BF16_PARAM, _lib.BF16_GRAD
    st, buf, blocks = _pack_ex([_tx(1 << 40, 2048, BP), _tx(2 << 40, 1, BG), _tx(3 << 40, 5, BP | BG)])
    assert st == OK and blocks == 2 + 1 + 1
    assert [struct.unpack_from("<i", buf, 64 * i + 52)[0] for i in range(3)] == [BP, BG, BP | BG]
    # bf16 buffers need 2-byte alignment, and 8 bytes for the vector path
    e = _lib.AdamWTensorEx((1 << 40) + 8, 2 << 40, 3 << 40, 4 << 40, 100, BP, 0)
    st, buf, _ = _pack_ex([e])  # bf16 param 8-aligned, fp32 buffers 16-aligned: vector path
    assert st == OK and struct.unpack_from("<i", buf, 48)[0] == 1
    st, buf, _ = _pack_ex([_tx((1 << 40) + 2, 100, BP | BG, pstep=(1 << 30) + 2)])
    assert st == ALIGN  # exp_avg would be 2-byte aligned (fp32 needs 4)
    e = _lib.AdamWTensorEx((1 << 40) + 2, 2 << 40, 3 << 40, 4 << 40, 100, BP, 0)
    st, buf, _ = _pack_ex([e])
    assert st == OK and struct.unpack_from("<i", buf, 48)[0] == 0  # bf16 param 2-aligned: scalar path
    e = _lib.AdamWTensorEx((1 << 40) + 1, 2 << 40, 3 << 40, 4 << 40, 100, BP, 0)
    assert _pack_ex([e])[0] == ALIGN


def test_adamw_pack_ex_rejects():
    BP = _lib.BF16_PARAM
    assert _pack_ex([_tx(1 << 40, 10, 4)])[0] == HYPER  # unknown flag bit
    e = _lib.AdamWTensorEx(1 << 40, 2 << 40, 3 << 40, 4 << 40, 10, 0, 1)
    assert _pack_ex([e])[0] == HYPER  # reserved != 0
    # overlap computed with the bf16 size: a bf16 param of 100 elements ends 200 bytes on
    e = _lib.AdamWTensorEx(1 << 40, (1 << 40) + 200, 3 << 40, 4 << 40, 100, BP, 0)
    assert _pack_ex([e])[0] == OK
    e = _lib.AdamWTensorEx(1 << 40, (1 << 40) + 196, 3 << 40, 4 << 40, 100, BP, 0)
    assert _pack_ex([e])[0] == ALIAS


@pytest.mark.parametrize("bad,code", [
    (_lib.AdamWTensor(0, 1 << 40, 2 << 40, 3 << 40, 10), NULL),
    (_lib.AdamWTensor(1 << 40, 2 << 40, 3 << 40, 4 << 40, -1), NUMEL),
    (_lib.AdamWTensor((1 << 40) + 2, 2 << 40, 3 << 40, 4 << 40, 10), ALIGN),
    (_lib.AdamWTensor(1 << 40, (1 << 40) + 8, 3 << 40, 4 << 40, 10), ALIAS),  # param overlaps grad
    (_lib.AdamWTensor(1 << 40, 2 << 40, 3 << 40, (3 << 40) + 16, 10), ALIAS),  # exp_avg overlaps exp_avg_sq
])
def test_adamw_pack_rejects(bad, code):
    st, _, _ = _pack([bad])
    assert st == code


def test_adamw_pack_rejects_aliasing_across_tensors():
    """One launch updates every tensor of a table at once: what a tensor writes
    must stay clear of what any other tensor reads or writes (a parameter
    listed twice included); gradients may be shared.  Both packers."""
    BP = _lib.BF16_PARAM
    a = _t(1 << 40, 1000)  # 4000-byte buffers
    assert _pack([a, _t(2 << 40, 1000)])[0] == OK
    a_bufs = [a.param, a.grad, a.exp_avg, a.exp_avg_sq]
    for j, d in ((0, 0), (1, 8), (2, 4000 - 16), (3, 64)):  # somewhere in each of a's buffers
        for k in (0, 2, 3):  # one of the second tensor's written buffers lands there
            f = [(2 << 40) + i * (1 << 30) for i in range(4)]
            f[k] = a_bufs[j] + d
            assert _pack([a, _lib.AdamWTensor(*f, 1000)])[0] == ALIAS, (j, k)
            assert _pack_ex([_lib.AdamWTensorEx(*f, 1000, 0, 0), _tx(1 << 40, 1000, 0)])[0] == ALIAS, (j, k)
    b = _t(2 << 40, 1000)
    b.grad = a.grad  # a shared gradient is only read
    assert _pack([a, b])[0] == OK
    b.grad = a.param + 3996  # reads the last element a writes
    assert _pack([a, b])[0] == ALIAS
    b.grad = a.param + 4000  # the next byte on: clear
    assert _pack([a, b])[0] == OK
    assert _pack([a, _t(1 << 40, 1000)])[0] == ALIAS  # the same tensor twice
    # extents per element type: a bf16 parameter of 1000 elements ends 2000 bytes on
    other = [(2 << 40) + i * (1 << 30) for i in range(4)]
    for grad, code in (((1 << 40) + 2000, OK), ((1 << 40) + 1996, ALIAS)):
        e = _lib.AdamWTensorEx(other[0], grad, other[2], other[3], 1000, 0, 0)
        assert _pack_ex([_tx(1 << 40, 1000, BP), e])[0] == code


def test_adamw_pack_small_table_and_counts():
    lib = _lib.load()
    arr = (_lib.AdamWTensor * 2)(_t(1 << 40, 10), _t(2 << 40, 10))
    buf = (ctypes.c_uint8 * 64)()
    blocks = ctypes.c_int64()
    assert lib.mamw_adamw_table_pack(arr, 2, buf, 64, ctypes.byref(blocks)) == TABLE
    assert lib.mamw_adamw_table_pack(arr, -1, buf, 64, ctypes.byref(blocks)) == COUNT
    assert lib.mamw_adamw_table_bytes(-5, ctypes.byref(ctypes.c_size_t())) == COUNT


def test_adamw_launch_validation_before_hip():
    lib = _lib.load()
    args = (3e-4, 0.1, 0.05, 0.9, 0.95, 0.1, 1e-8, None)
    assert lib.mamw_adamw_mt_step(None, 1, 5, *args) == NULL
    assert lib.mamw_adamw_mt_step(1 << 40 | 8, 1, 5, *args) == ALIGN
    assert lib.mamw_adamw_mt_step(1 << 40, 1, -1, *args) == NUMEL
    assert lib.mamw_adamw_mt_step(1 << 40, 0, 5, *args) == COUNT
    assert lib.mamw_adamw_mt_step(None, 0, 0, *args) == OK  # nothing to do: no launch
    assert lib.mamw_adamw_tensor_step(None, None, None, None, 0, *args) == OK
    assert lib.mamw_adamw_tensor_step(None, 1 << 40, 2 << 40, 3 << 40, 7, *args) == NULL


# ---- Muon workspace and validation -------------------------------------------------

def _ws(batch, rows, cols, steps=5):
    n = ctypes.c_size_t()
    st = _lib.load().mamw_muon_workspace_bytes(batch, rows, cols, steps, ctypes.byref(n))
    return st, n.value


def _rup(x, t):
    return (x + t - 1) // t * t


def _tile(batch, m, n):
    """The documented tile rule: 256 from m = 2048; from m = 1024 for batches
    of 8 or more when the 256 padding adds at most 1/16 to the 128 padding."""
    if m >= 2048:
        return 256
    if m >= 1024 and batch >= 8 and _rup(m, 256) * _rup(n, 256) * 16 <= _rup(m, 128) * _rup(n, 128) * 17:
        return 256
    return 128


@pytest.mark.parametrize("batch,rows,cols,steps", [(1, 768, 3072, 5), (24, 3072, 768, 5), (16, 14336, 4096, 5),
                                                   (3, 100, 37, 1), (2, 5, 7, 0), (1, 32768, 32768, 5),
                                                   (16, 1024, 2100, 5), (4, 1024, 2100, 5), (16, 1100, 4096, 5),
                                                   (1, 8192, 130816, 5), (1, 130816, 8192, 5), (1, 8192, 131072, 5)])
def test_workspace_layout(batch, rows, cols, steps):
    """X (bf16, mp x np per matrix) is kept only in a row-major workspace (a
    matrix of 2^31 bytes or more); then X^T twice, A and B, the prep partial
    sums and the norms, each region 256-byte aligned.  8192 x 130816 is the
    largest k-blocked matrix of its row count (2^31 - 2^22 bytes); 8192 x
    131072 is row-major."""
    st, got = _ws(batch, rows, cols, steps)
    assert st == OK
    m, n = min(rows, cols), max(rows, cols)
    tile = _tile(batch, m, n)
    mp, np_ = _rup(m, tile), _rup(n, tile)
    a = lambda x: _rup(x, 256)  # noqa: E731
    xe = batch * mp * np_ * 2
    ae = batch * mp * mp * 2
    rowmajor = mp * np_ * 2 >= 1 << 31
    expect = (a(xe) if rowmajor else 0) + a(xe) + (a(xe) if steps >= 2 else 0) + (2 * a(ae) if steps >= 1 else 0)
    expect += a(batch * (mp // 64) * (np_ // 64) * 4) + a(batch * 4)
    assert got == expect


@pytest.mark.parametrize("args,code", [((0, 10, 10, 5), COUNT), ((33, 10, 10, 5), COUNT), ((1, 0, 10, 5), SHAPE),
                                       ((1, 10, -3, 5), SHAPE), ((1, 10, 10, 100), HYPER), ((1, 10, 10, -1), HYPER),
                                       ((1, 1 << 21, 10, 5), SHAPE)])
def test_workspace_rejects(args, code):
    assert _ws(*args)[0] == code


def _mats(specs):
    arr = (_lib.MuonMatrix * len(specs))()
    for i, (r, c) in enumerate(specs):
        base = (i + 1) << 36
        arr[i] = _lib.MuonMatrix(base, base + (1 << 34), base + (2 << 34), None, r, c, 1e-3, 0)
    return arr


def _step(arr, n, ws=1 << 45, ws_bytes=1 << 40, steps=5):
    return _lib.load().mamw_muon_step(arr, n, 1e-3, 0.1, 0.95, 1, 3.4445, -4.775, 2.0315, steps, 1e-7, ws,
                                      ws_bytes, None)


def test_muon_step_rejects_before_hip():
    arr = _mats([(256, 512), (512, 300)])
    assert _step(arr, 2) == SHAPE  # {256,512} vs {300,512}
    arr = _mats([(256, 512), (512, 256)])
    assert _step(arr, 2, ws=None) == WS
    assert _step(arr, 2, ws=(1 << 45) + 64) == WS  # not 256-byte aligned
    assert _step(arr, 2, ws_bytes=1000) == WS
    assert _step(arr, 0) == COUNT
    assert _step(arr, 2, steps=100) == HYPER
    arr[1].flags = 4  # not a MAMW_BF16_* bit
    assert _step(arr, 2) == HYPER
    arr = _mats([(256, 512), (512, 256)])
    arr[1].param = arr[0].param  # two entries update the same parameter
    assert _step(arr, 2) == ALIAS
    # across entries, whatever one entry writes must stay clear of what another reads or writes
    for field_i, field_j in (("momentum", "grad"), ("param", "momentum"), ("grad", "param"), ("update", "param"),
                             ("momentum", "update")):
        arr = _mats([(256, 512), (512, 256), (256, 512)])
        for a in arr:
            a.update = a.param + (3 << 34)
        setattr(arr[2], field_i, getattr(arr[1], field_j) + 64)
        assert _step(arr, 3) == ALIAS, (field_i, field_j)
    arr = _mats([(256, 512), (512, 256), (300, 512)])
    arr[1].grad = arr[0].grad  # two entries reading one gradient is fine: entries 0 and 1 pass,
    assert _step(arr, 3) == SHAPE  # and validation stops at entry 2's shape
    arr = _mats([(256, 512)])
    arr[0].grad = arr[0].param + 4
    assert _step(arr, 1) == ALIAS
    arr = _mats([(256, 512)])
    arr[0].momentum = (1 << 45) + 4096  # inside the workspace
    assert _step(arr, 1) == ALIAS
    arr = _mats([(256, 512)])
    arr[0].param = None
    assert _step(arr, 1) == NULL
    arr = _mats([(256, 512)])
    arr[0].update = arr[0].param + 2
    assert _step(arr, 1) == ALIGN


def test_muon_step_noalloc_rejects_before_hip():
    """The no-allocation entry point validates like mamw_muon_step, and a batch
    whose workspace exceeds the library's static scratch is rejected with
    MAMW_ERR_SCRATCH, all before any HIP call."""
    lib = _lib.load()

    def call(arr, n, steps=5):
        return lib.mamw_muon_step_noalloc(arr, n, 1e-3, 0.1, 0.95, 1, 3.4445, -4.775, 2.0315, steps, 1e-7, None)

    assert call(_mats([(4096, 14336)]), 1) == SCRATCH  # one 4096 x 14336 matrix needs 288 MiB
    assert call(_mats([(4096, 4096)] * 2), 2) == SCRATCH
    assert call(_mats([(1024, 4096)] * 13), 13) == SCRATCH
    assert call(_mats([(256, 512), (512, 300)]), 2) == SHAPE
    assert call(_mats([(256, 512)]), 0) == COUNT
    assert call(_mats([(256, 512)]), 1, steps=100) == HYPER
    arr = _mats([(256, 512)])
    arr[0].grad = arr[0].param + 4
    assert call(arr, 1) == ALIAS
    assert call(None, 1) == NULL
    assert "scratch" in lib.mamw_strerror(SCRATCH).decode()
    # the documented fits (both orientations)
    for shape, k in (((4096, 4096), 1), ((1024, 4096), 12), ((768, 3072), 22), ((3072, 768), 22),
                     ((768, 2304), 28), ((768, 768), 32)):
        n = ctypes.c_size_t()
        assert lib.mamw_muon_workspace_bytes(k, shape[0], shape[1], 5, ctypes.byref(n)) == OK
        assert n.value <= 256 << 20, (shape, k, n.value)
        if k < 32:  # and the documented figure is the largest batch that fits
            assert lib.mamw_muon_workspace_bytes(k + 1, shape[0], shape[1], 5, ctypes.byref(n)) == OK
            assert n.value > 256 << 20, (shape, k + 1, n.value)


def test_ns_blocks_validation():
    lib = _lib.load()
    assert lib.mamw_ns_gram(1 << 40, 2 << 40, 1, 100, 64, None) == SHAPE
    assert lib.mamw_ns_gram(1 << 40, 2 << 40, 1, 128, 96, None) == SHAPE
    assert lib.mamw_ns_gram(None, 2 << 40, 1, 128, 64, None) == NULL
    assert lib.mamw_ns_gram((1 << 40) + 2, 2 << 40, 1, 128, 64, None) == ALIGN
    assert lib.mamw_ns_poly(1 << 40, 1 << 40, 1, 128, -4.775, 2.03, None) == ALIAS
    assert lib.mamw_ns_update(1 << 40, 2 << 40, 3 << 40, 4 << 40, 3 << 40, 1, 128, 256, 3.44, None) == ALIAS
    assert lib.mamw_ns_update(1 << 40, 2 << 40, 3 << 40, 4 << 40, None, 1, 128, 200, 3.44, None) == SHAPE
    assert lib.mamw_transpose_bf16(1 << 40, 1 << 40, 1, 4, 4, None) == ALIAS
    assert lib.mamw_transpose_bf16(1 << 40, (1 << 40) + 16, 1, 4, 4, None) == ALIAS  # partial overlap
    assert lib.mamw_transpose_bf16(1 << 40, 2 << 40, 0, 4, 4, None) == COUNT


def test_ns_blocks_reject_overlapping_buffers():
    """Operands, epilogue sources and outputs of the standalone GEMMs that would
    race are rejected by byte-range overlap before any HIP call."""
    lib = _lib.load()
    m, k = 256, 512
    X = 1 << 40
    # Gram: A inside X, or X starting inside A
    assert lib.mamw_ns_gram(X, X + 2 * m * 64, 1, m, k, None) == ALIAS
    assert lib.mamw_ns_gram(X + 1024, X, 1, m, k, None) == ALIAS
    # polynomial: B overlapping A partly
    assert lib.mamw_ns_poly(X, X + 2 * m * m - 16, 1, m, -4.775, 2.03, None) == ALIAS
    assert lib.mamw_ns_poly(X, X + 2 * 2 * m * m - 16, 2, m, -4.775, 2.03, None) == ALIAS  # batch extent
    # update: out over B, out over XT, out_t over B / XT / out
    n = 512
    B, XT, out, out_t = 1 << 40, 2 << 40, 3 << 40, 4 << 40
    assert lib.mamw_ns_update(B, out, XT, B + 64, None, 1, m, n, 3.44, None) == ALIAS
    assert lib.mamw_ns_update(B, out, XT, XT + 2 * n * m - 16, None, 1, m, n, 3.44, None) == ALIAS
    assert lib.mamw_ns_update(B, out, XT, out, B, 1, m, n, 3.44, None) == ALIAS
    assert lib.mamw_ns_update(B, out, XT, out, XT + 4096, 1, m, n, 3.44, None) == ALIAS
    assert lib.mamw_ns_update(B, out, XT, out, out + 2 * m * n - 16, 1, m, n, 3.44, None) == ALIAS


def test_profiler_without_launches():
    _lib.prof_start()
    _lib.prof_stop()
    assert _lib.prof_collect() == []
    lib = _lib.load()
    assert lib.mamw_prof_kernel_name(0).decode() == "adamw_mt_kernel"
    assert lib.mamw_prof_kernel_name(99).decode() == "unknown"


def test_adamw_amp_launch_validation_before_hip():
    """mamw_adamw_mt_step_amp rejects its arguments on the host before its
    first launch (the bias-correction kernel), so nothing here touches a GPU."""
    lib = _lib.load()
    step = 1 << 40  # never dereferenced: every call below is rejected or launches nothing
    hp = (3e-4, 0.9, 0.95, 0.1, 1e-8)
    assert lib.mamw_adamw_mt_step_amp(1 << 40, 1, 5, *hp, None, None, None, None) == NULL
    assert lib.mamw_adamw_mt_step_amp(None, 1, 5, *hp, step, None, None, None) == NULL
    assert lib.mamw_adamw_mt_step_amp(1 << 40 | 8, 1, 5, *hp, step, None, None, None) == ALIGN
    assert lib.mamw_adamw_mt_step_amp(1 << 40, 1, -1, *hp, step, None, None, None) == NUMEL
    assert lib.mamw_adamw_mt_step_amp(1 << 40, 0, 5, *hp, step, None, None, None) == COUNT
    assert lib.mamw_adamw_mt_step_amp(1 << 40, -1, 5, *hp, step, None, None, None) == COUNT
    assert lib.mamw_adamw_mt_step_amp(None, 0, 0, *hp, step, None, None, None) == OK  # nothing to do
    # beyond the grid limit: rejected before the bias kernel would be launched
    assert lib.mamw_adamw_mt_step_amp(1 << 40, 1, 1 << 31, *hp, step, None, None, None) == NUMEL
    assert lib.mamw_adamw_mt_step(1 << 40, 1, 1 << 31, 3e-4, 0.1, 0.05, 0.9, 0.95, 0.1, 1e-8, None) == NUMEL
