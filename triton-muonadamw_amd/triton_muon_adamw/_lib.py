"""ctypes binding of ``libmuonadamw_amd.so`` (the C ABI in include/muonadamw_amd.h).

The library is loaded once, from next to this file.  There is no fallback:
if the library is missing every optimizer step raises, so a run never
silently computes on another path.

Status codes map to exceptions: negative (argument rejected on the host) ->
``ValueError``; positive (a hipError_t) -> ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmuonadamw_amd.so")
ABI_VERSION = 5
MUON_MAX_BATCH = 32
BF16_PARAM = 0x1  # MAMW_BF16_PARAM
BF16_GRAD = 0x2   # MAMW_BF16_GRAD


class AdamWTensor(ctypes.Structure):
    """``mamw_adamw_tensor``."""

    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("exp_avg", c_void_p),
        ("exp_avg_sq", c_void_p),
        ("numel", c_int64),
    ]


class AdamWTensorEx(ctypes.Structure):
    """``mamw_adamw_tensor_ex``."""

    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("exp_avg", c_void_p),
        ("exp_avg_sq", c_void_p),
        ("numel", c_int64),
        ("flags", c_int32),
        ("reserved", c_int32),
    ]


class MuonMatrix(ctypes.Structure):
    """``mamw_muon_matrix``."""

    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("momentum", c_void_p),
        ("update", c_void_p),
        ("rows", c_int64),
        ("cols", c_int64),
        ("scaled_lr", c_float),
        ("flags", c_int32),
    ]


class ProfRecord(ctypes.Structure):
    """``mamw_prof_record``."""

    _fields_ = [
        ("kernel", c_int32),
        ("variant", c_int32),
        ("flops", c_double),
        ("bytes", c_double),
        ("ms", c_float),
        ("pad", c_int32),
    ]


_PROTOTYPES = {
    "mamw_abi_version": (c_int, []),
    "mamw_strerror": (c_char_p, [c_int]),
    "mamw_adamw_tensor_step": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_float, c_float, c_float, c_float,
         c_float, c_float, c_float, c_void_p],
    ),
    "mamw_adamw_table_bytes": (c_int, [c_int, POINTER(c_size_t)]),
    "mamw_adamw_table_pack": (c_int, [POINTER(AdamWTensor), c_int, c_void_p, c_size_t, POINTER(c_int64)]),
    "mamw_adamw_table_pack_ex": (c_int, [POINTER(AdamWTensorEx), c_int, c_void_p, c_size_t, POINTER(c_int64)]),
    "mamw_adamw_mt_step": (
        c_int,
        [c_void_p, c_int, c_int64, c_float, c_float, c_float, c_float, c_float, c_float, c_float,
         c_void_p],
    ),
    "mamw_adamw_mt_step_amp": (
        c_int,
        [c_void_p, c_int, c_int64, c_float, c_double, c_double, c_float, c_float, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "mamw_muon_workspace_bytes": (c_int, [c_int, c_int64, c_int64, c_int, POINTER(c_size_t)]),
    "mamw_muon_step": (
        c_int,
        [POINTER(MuonMatrix), c_int, c_double, c_double, c_double, c_int, c_float, c_float, c_float,
         c_int, c_float, c_void_p, c_size_t, c_void_p],
    ),
    "mamw_muon_step_noalloc": (
        c_int,
        [POINTER(MuonMatrix), c_int, c_double, c_double, c_double, c_int, c_float, c_float, c_float,
         c_int, c_float, c_void_p],
    ),
    "mamw_muon_step_amp": (
        c_int,
        [POINTER(MuonMatrix), c_int, c_double, c_double, c_double, c_int, c_float, c_float, c_float,
         c_int, c_float, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p],
    ),
    "mamw_ns_gram": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_int64, c_void_p]),
    "mamw_ns_poly": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_float, c_float, c_void_p]),
    "mamw_ns_update": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_float, c_void_p],
    ),
    "mamw_transpose_bf16": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_int64, c_void_p]),
    "mamw_prof_start": (c_int, []),
    "mamw_prof_stop": (c_int, []),
    "mamw_prof_collect": (c_int, [POINTER(ProfRecord), c_int, POINTER(c_int)]),
    "mamw_prof_kernel_name": (c_char_p, [c_int]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the library (once) and declare every prototype."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH.name} is not built; run __graft_entry__.build() "
            "(or python -m triton_muon_adamw._build). MuonAdamW has no fallback path.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mamw_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH.name} ABI {lib.mamw_abi_version()} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def strerror(status: int) -> str:
    return load().mamw_strerror(status).decode()


def check(status: int, what: str) -> None:
    """Raise for a non-zero status returned by ``what``."""
    if status == 0:
        return
    msg = f"{what}: {strerror(status)} (status {status})"
    if status < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_flag(t: torch.Tensor, bit: int, name: str) -> int:
    """``bit`` when ``t`` holds bf16, 0 for fp32; other dtypes are an error."""
    if t.dtype == torch.bfloat16:
        return bit
    if t.dtype == torch.float32:
        return 0
    raise TypeError(f"{name} must be float32 or bfloat16 (got {t.dtype})")


def require_gpu_tensor(t: torch.Tensor, name: str) -> None:
    """The kernels run on ROCm devices only; CPU tensors are an error."""
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; MuonAdamW's HIP kernels need tensors on a ROCm GPU "
            "(there is no CPU path)")


def layout_key(p: torch.Tensor) -> tuple:
    """What a cached launch plan assumes of a parameter and its gradient:
    addresses, element types and layouts.  A step whose parameters differ in
    any of these builds a new plan (e.g. ``p.data`` replaced by a view that
    starts at the same address with another shape)."""
    g = p.grad
    return (id(p), p.data_ptr(), p.dtype, p.shape, p.stride(), g.data_ptr(), g.dtype, g.shape, g.stride())


def check_not_capturing(branch: str) -> None:
    """Launch plans and device step counters are made by eager steps only: a
    graph replays the pointers, scalars and table upload recorded at capture."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"{branch}: a launch plan or step counter would be created during graph capture; take one eager "
            "step first and keep the .grad tensors static between capture and replay (copy new gradients "
            "into them)")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (0 = null stream)."""
    return torch.cuda.current_stream(device).cuda_stream


_HIP_STREAM_NON_BLOCKING = 1
# Streams of threads that have exited, per device index, for reuse by new threads.
_free_side_streams: dict[int, list] = {}
_side_streams_lock = threading.Lock()
_thread_side_streams = threading.local()


class _ThreadStreams:
    """One thread's side streams per device; when the thread ends (its
    thread-local storage is released) they return to the free list."""

    def __init__(self):
        self.by_device: dict[int, list] = {}

    # The lock and the free list are bound as defaults: at interpreter exit
    # the main thread's storage can outlive the module's globals.
    def __del__(self, _lock=_side_streams_lock, _free=_free_side_streams):
        with _lock:
            for idx, streams in self.by_device.items():
                _free.setdefault(idx, []).extend(streams)


def side_streams(device: torch.device, count: int) -> list:
    """``count`` streams of the library's own on ``device`` for shape classes
    that run beside the caller's stream, per calling thread and device.  Per
    thread: a thread that captures a step into a graph forks these streams
    into the capture, so an optimizer stepping eagerly on another thread must
    not queue work on the same streams meanwhile.  A thread's streams are
    created on first use and go back to a free list when the thread ends, for
    the next thread to take (none is destroyed: at most as many exist as
    threads have used them at once).

    They come from hipStreamCreateWithFlags(hipStreamNonBlocking), looked up
    through this library's handle (so from the HIP runtime the library and
    torch share), not from torch's stream pool: the runtime gives a new stream
    the least used of its hardware queues (GPU_MAX_HW_QUEUES of them, 4 by
    default), which keeps up to GPU_MAX_HW_QUEUES - 1 of these streams off the
    queue of the null stream and off each other's.  Which queue a pool stream
    shares depends on how many the pool has handed out before (measured: one
    small Muon step 5.0 or 5.6 ms depending on that history).  Non-blocking:
    the legacy null stream does not wait for them, nor they for it."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    mine = getattr(_thread_side_streams, "streams", None)
    if mine is None:
        mine = _thread_side_streams.streams = _ThreadStreams()
    have = mine.by_device.setdefault(idx, [])
    if len(have) < count:
        with _side_streams_lock:
            free = _free_side_streams.get(idx, [])
            while free and len(have) < count:
                have.append(free.pop())
    if len(have) < count:
        create = load().hipStreamCreateWithFlags
        create.restype = c_int
        create.argtypes = [POINTER(c_void_p), ctypes.c_uint]
        with torch.cuda.device(idx):
            while len(have) < count:
                s = c_void_p()
                st = create(ctypes.byref(s), _HIP_STREAM_NON_BLOCKING)
                if st != 0 or not s.value:
                    raise RuntimeError(f"hipStreamCreateWithFlags failed on device {idx} (hipError {st})")
                have.append(torch.cuda.ExternalStream(s.value, device=torch.device("cuda", idx)))
    return have[:count]


def prof_start() -> None:
    """Start timing every kernel launch of the library (HIP events per dispatch)."""
    check(load().mamw_prof_start(), "mamw_prof_start")


def prof_stop() -> None:
    check(load().mamw_prof_stop(), "mamw_prof_stop")


def prof_collect() -> list[dict]:
    """Wait for the recorded launches and return one dict per launch, in launch order."""
    lib = load()
    count = c_int(0)
    st = lib.mamw_prof_collect(None, 0, ctypes.byref(count))
    if st not in (0, -8):
        check(st, "mamw_prof_collect")
    n = count.value
    if n == 0:
        return []
    recs = (ProfRecord * n)()
    check(lib.mamw_prof_collect(recs, n, ctypes.byref(count)), "mamw_prof_collect")
    return [
        {"kernel": lib.mamw_prof_kernel_name(r.kernel).decode(), "variant": r.variant, "flops": r.flops,
         "bytes": r.bytes, "ms": r.ms}
        for r in recs[: count.value]
    ]
