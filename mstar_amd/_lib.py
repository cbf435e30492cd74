"""ctypes binding of the gfx950 C ABI declared in ``include/mstar_amd.h``.

The library is built in-tree by ``mstar_amd.build`` (``libmstar_amd.so`` next to
this file).  There is no fallback: if the library is missing or was built for
a different ABI version, :func:`lib` raises, and every caller fails loudly.
``torch`` is imported before the library is loaded so that the dynamic linker
binds our ``libamdhip64.so.7`` dependency to torch's already-loaded HIP
runtime: torch tensors and these kernels then share one HIP context.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

LIB_PATH = Path(__file__).resolve().parent / "libmstar_amd.so"
ABI_VERSION = 4

# dtype codes (mstar_amd.h)
MI_BF16 = 0
MI_F16 = 1
MI_F32 = 2
MI_FP8_E4M3 = 3
MI_I32 = 4
MI_I64 = 5

MI_OK = 0
MI_ERR_UNSUPPORTED = -2

TORCH_TO_MI = {
    torch.bfloat16: MI_BF16,
    torch.float16: MI_F16,
    torch.float32: MI_F32,
    torch.float8_e4m3fn: MI_FP8_E4M3,
}


class MiPagedKV(ctypes.Structure):
    """Mirror of ``mi_paged_kv`` (mstar_amd.h)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_pages", ctypes.c_int64),
        ("page_stride", ctypes.c_int64),
        ("kv_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
    ]


class MiKvPool(ctypes.Structure):
    """Mirror of ``mi_kv_pool`` (mstar_amd.h)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("layer_stride", ctypes.c_int64),
        ("page_stride", ctypes.c_int64),
        ("kv_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("num_pages", ctypes.c_int64),
        ("num_layers", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

# name -> (restype, argtypes); must match include/mstar_amd.h exactly.
SIGNATURES = {
    "mi_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mi_abi_version": (ctypes.c_int, []),
    "mi_pack": (ctypes.c_int, [_P, _P, _P, _P, _I32, _P, _I64, _P, _P, _I32, _P, _P, _P, _P, _P, _I32, _P]),
    "mi_pack_plan": (
        ctypes.c_int,
        [_P, _P, _P, _P, _I32, _P, _I64, _P, _P, _I32, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _I64, _P],
    ),
    "mi_pack_plan_host": (
        ctypes.c_int,
        [_P, _I32, _I32, _P, _I64, _I32, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _P, _I64, _P],
    ),
    "mi_block_table_update": (ctypes.c_int, [_P, _I64, _P, _P, _P, _I32, _P]),
    "mi_decode_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32]),
    "mi_decode_plan": (ctypes.c_int, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _I64, _P]),
    "mi_decode_run": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_decode_attend": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_decode_merge": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_decode_noalloc": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _F32,
         _P, _I64, _I64, _P, _P],
    ),
    "mi_kv_append": (
        ctypes.c_int,
        [ctypes.POINTER(MiPagedKV), _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _P, _I64, _I32, _P, _P],
    ),
    "mi_prefill_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "mi_prefill_short_rows": (_I32, [_I32, _I32, _I32, _I32]),
    "mi_prefill_plan": (
        ctypes.c_int,
        [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _I32, _P, _I64, _P],
    ),
    "mi_prefill_run": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_prefill_short": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_prefill_tiles": (
        ctypes.c_int,
        [_P, _I32, _I64, _I64, ctypes.POINTER(MiPagedKV), _P, _P, _P, _P, _I32, _I32, _I32, _I32, _F32,
         _P, _I64, _P, _I64, _I64, _P],
    ),
    "mi_rope_positions": (ctypes.c_int, [_P, _P, _I32, _P, _I32, _P]),
    "mi_copy_pages": (ctypes.c_int, [_P, _I64, _I32, _I64, _I64, _I64, _P, _P, _I32, _P]),
    "mi_kv_copy_tokens": (
        ctypes.c_int,
        [ctypes.POINTER(MiKvPool), ctypes.POINTER(MiKvPool), _P, _P, _P, _P, _I32, _I32, _I32, _P],
    ),
    "mi_kv_wire_pack": (
        ctypes.c_int,
        [ctypes.POINTER(MiKvPool), _P, _P, _P, _P, _I32, _I32, _I32, _P, _I64, _P],
    ),
    "mi_kv_wire_unpack": (
        ctypes.c_int,
        [_P, _I64, ctypes.POINTER(MiKvPool), _P, _P, _P, _P, _I32, _I32, _I32, _P],
    ),
    "mi_hbm_read": (ctypes.c_int, [_P, _I64, _P, _I32, _P]),
    "mi_rope_apply": (
        ctypes.c_int,
        [_P, _I64, _I64, _I32, _P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _I32, _I32, _I32, _F32, _F32,
         _I32, _F32, _F32, _F32, _P],
    ),
    "mi_rope_append": (
        ctypes.c_int,
        [_P, _I64, _I64, _I32, _P, _I64, _I64, _P, _I64, _I64, _I32, _I32, ctypes.POINTER(MiPagedKV), _P, _P,
         _I64, _I32, _P, _I32, _P, _I32, _I32, _I32, _F32, _F32, _I32, _F32, _F32, _F32, _P],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the gfx950 kernels first "
                "(python -m mstar_amd.build). There is no CPU fallback."
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.mi_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a nonzero C status to an exception."""
    if status != MI_OK:
        text = lib().mi_status_string(status).decode()
        if status == -1:
            raise ValueError(f"{what}: {text} (status {status})")
        raise RuntimeError(f"{what}: {text} (status {status})")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device | None = None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    if _raw_stream is not None and isinstance(device, torch.device) and device.index is not None:
        return _raw_stream(device.index)  # same value, without building a Stream object
    return torch.cuda.current_stream(device).cuda_stream


_memcpy_async = None


def memcpy_h2d_async(dst: int, src: int, nbytes: int, stream: int) -> None:
    """hipMemcpyAsync host -> device on ``stream`` (HIP runtime this library is bound to)."""
    global _memcpy_async
    if _memcpy_async is None:
        fn = lib().hipMemcpyAsync  # resolved through the library's own HIP runtime dependency
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
        _memcpy_async = fn
    rc = _memcpy_async(dst, src, nbytes, 1, stream)  # 1 = hipMemcpyHostToDevice
    if rc != 0:
        raise RuntimeError(f"hipMemcpyAsync failed with HIP error {rc}")


_event_fns = None


def _events_api():
    """hipEventCreateWithFlags / hipEventRecord / hipEventSynchronize of the
    HIP runtime this library is bound to."""
    global _event_fns
    if _event_fns is None:
        h = lib()
        create, record, sync = h.hipEventCreateWithFlags, h.hipEventRecord, h.hipEventSynchronize
        create.restype = record.restype = sync.restype = ctypes.c_int
        create.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        record.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        sync.argtypes = [ctypes.c_void_p]
        _event_fns = (create, record, sync)
    return _event_fns


def _event_create(device: torch.device) -> int:
    """A timing-free HIP event on ``device`` (kept for the life of the process)."""
    create = _events_api()[0]
    ev = ctypes.c_void_p()
    with torch.cuda.device(device):
        rc = create(ctypes.byref(ev), 2)  # 2 = hipEventDisableTiming
    if rc != 0:
        raise RuntimeError(f"hipEventCreateWithFlags failed with HIP error {rc}")
    return ev.value


PACK_HOST_META = 768  # MI_PACK_HOST_META: int32 values of step metadata always passed as a kernel argument
PACK_HOST_META_MAX = 4096  # MI_PACK_HOST_META_MAX: up to this many when the step fits the argument's compact form


class PinnedUploader:
    """Small int32 host arrays to the device through two pinned staging buffers.

    Buffers alternate, so writing this call's data waits only for the copy
    issued two calls ago; the copy is one hipMemcpyAsync on the current
    stream into a fresh device tensor.  The staging buffers are never handed
    back to torch's pinned-memory cache while a copy from them may be
    pending (the raw copy records nothing there): use the per-device
    instance from :func:`uploader`, which lives for the process, and a buffer
    is only replaced after its last copy has finished.
    """

    def __init__(self, device: torch.device):
        self.device = torch.device(device)
        self._bufs: list = [None, None]
        self._events: list = [None, None]
        self._i = 0
        self._lock = threading.Lock()

    def upload(self, arr) -> torch.Tensor:
        n = int(arr.size)
        with self._lock:
            i = self._i
            self._i ^= 1
            ev = self._events[i]
            _, record, sync = _events_api()
            if ev is not None:
                rc = sync(ev)  # the copy that last read this buffer is done
                if rc != 0:
                    raise RuntimeError(f"hipEventSynchronize failed with HIP error {rc}")
            buf = self._bufs[i]
            if buf is None or buf[1].size < n:
                t = torch.empty(max(n, 4096), dtype=torch.int32, pin_memory=True)
                buf = self._bufs[i] = (t, t.numpy(), t.data_ptr())
            buf[1][:n] = arr
            dev = torch.empty(max(n, 1), dtype=torch.int32, device=self.device)
            stream = stream_ptr(self.device)
            if n:
                memcpy_h2d_async(dev.data_ptr(), buf[2], 4 * n, stream)
            if ev is None:
                ev = self._events[i] = _event_create(self.device)
            rc = record(ev, stream)
            if rc != 0:
                raise RuntimeError(f"hipEventRecord failed with HIP error {rc}")
        return dev if n == dev.shape[0] else dev[:n]


_uploaders: dict = {}
_uploaders_lock = threading.Lock()


def uploader(device) -> PinnedUploader:
    """The process-wide :class:`PinnedUploader` of ``device``."""
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    with _uploaders_lock:
        u = _uploaders.get(d)
        if u is None:
            u = _uploaders[d] = PinnedUploader(d)
    return u


_desc_cache: dict = {}


def _scale_key(s: torch.Tensor | None):
    if s is None:
        return None
    return (s.data_ptr(), s.dtype, s.numel(), s.is_contiguous(), s.device)


def paged_kv_desc(kv_cache_layer: torch.Tensor, k_scale: torch.Tensor | None = None,
                  v_scale: torch.Tensor | None = None) -> MiPagedKV:
    """Describe one KV layer ``[max_pages, 2, page_size, num_kv_heads, head_dim]``.

    Descriptors are kept by everything they are built and checked from
    (address, shape, strides, dtype, and the scales' address, dtype, size,
    layout and device), so a layer seen before costs one dictionary lookup.
    """
    key = (kv_cache_layer.data_ptr(), kv_cache_layer.shape, kv_cache_layer.stride(), kv_cache_layer.dtype,
           kv_cache_layer.device, _scale_key(k_scale), _scale_key(v_scale))
    d = _desc_cache.get(key)
    if d is None:
        d = _build_paged_kv_desc(kv_cache_layer, k_scale, v_scale)
        if len(_desc_cache) >= 256:
            _desc_cache.clear()
        _desc_cache[key] = d
    return d


def _build_paged_kv_desc(kv_cache_layer: torch.Tensor, k_scale: torch.Tensor | None,
                         v_scale: torch.Tensor | None) -> MiPagedKV:
    if kv_cache_layer.dim() != 5 or kv_cache_layer.shape[1] != 2:
        raise ValueError(
            f"kv_cache_layer must be [max_pages, 2, page_size, num_kv_heads, head_dim], got {tuple(kv_cache_layer.shape)}"
        )
    if kv_cache_layer.stride(4) != 1:
        raise ValueError("kv_cache_layer: head_dim must be contiguous")
    dt = TORCH_TO_MI.get(kv_cache_layer.dtype)
    if dt is None:
        raise ValueError(f"unsupported KV cache dtype {kv_cache_layer.dtype} (bf16, fp16, fp32 or float8_e4m3fn)")
    d = MiPagedKV()
    d.data = kv_cache_layer.data_ptr()
    d.dtype = dt
    d.page_size = kv_cache_layer.shape[2]
    d.num_kv_heads = kv_cache_layer.shape[3]
    d.head_dim = kv_cache_layer.shape[4]
    d.max_pages = kv_cache_layer.shape[0]
    d.page_stride = kv_cache_layer.stride(0)
    d.kv_stride = kv_cache_layer.stride(1)
    d.token_stride = kv_cache_layer.stride(2)
    d.head_stride = kv_cache_layer.stride(3)
    if dt == MI_FP8_E4M3:
        if k_scale is None or v_scale is None:
            raise ValueError("an fp8 KV cache needs per-head k_scale and v_scale tensors")
        for name, s in (("k_scale", k_scale), ("v_scale", v_scale)):
            if s.dtype != torch.float32 or s.numel() != d.num_kv_heads or not s.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 tensor of num_kv_heads elements")
            if s.device != kv_cache_layer.device:
                raise ValueError(f"{name} must live on the KV cache's device")
        d.k_scale = k_scale.data_ptr()
        d.v_scale = v_scale.data_ptr()
    else:
        d.k_scale = None
        d.v_scale = None
    return d
