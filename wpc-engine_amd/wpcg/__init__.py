"""Python binding of the wpcg C ABI (include/wpcg.h) over ctypes.

The classes mirror the reference's operator surface so tests read like the
reference's own (paths relative to the reference repository):
  WpcModelDataV4.open(dir)            wpc-runtime/src/wpc_weights_v4.rs:46-77
  WpcLinearV4(data, name, out, in)    wpc_weights_v4.rs:127-155
  Linear.matvec(x) -> y               wpc-runtime/src/weights.rs:17-22
  WpcEmbeddingV4.embed / .logits      wpc_weights_v4.rs:234-273
and the v3 twins. Every call goes through libwpcg.so; there is no CPU
fallback: if the library is missing, importing this module raises.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import re
import sys
import weakref

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
# WPCG_LIB names another build of the same library (the host-sanitizer build
# _build/asan/libwpcg_asan.so in tests/test_sanitize.py); by default lib/libwpcg.so.
LIB_PATH = os.environ.get("WPCG_LIB") or os.path.join(PKG_ROOT, "lib", "libwpcg.so")
HEADER = os.path.join(os.path.dirname(PKG_ROOT), "include", "wpcg.h")

OK, E_IO, E_FORMAT, E_SHAPE, E_NOTFOUND, E_DEVICE, E_ARG, E_NOMEM, E_UNSUPPORTED = range(9)
SCHEME_V3, SCHEME_V4 = 3, 4
MODE_EXACT, MODE_FAST = 0, 1
FAST_KERNEL_MFMA, FAST_KERNEL_VALU = 0, 1
ROUND_FMA, ROUND_TWO = 0, 1
DTYPE_F32, DTYPE_BF16, DTYPE_F32_SPLIT = 0, 1, 2

_ERR_NAMES = {0: "OK", 1: "E_IO", 2: "E_FORMAT", 3: "E_SHAPE", 4: "E_NOTFOUND", 5: "E_DEVICE",
              6: "E_ARG", 7: "E_NOMEM", 8: "E_UNSUPPORTED"}


class WpcgError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C {PKG_ROOT}` "
                          "or __graft_entry__.build()")
    return C.CDLL(LIB_PATH)


lib = _load()

_p = C.c_void_p
_pp = C.POINTER(C.c_void_p)
_u64 = C.c_uint64
_u64p = C.POINTER(C.c_uint64)
_SIGS = {
    "wpcg_last_error_string": (C.c_char_p, []),
    "wpcg_version": (C.c_char_p, []),
    "wpcg_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "wpcg_ctx_create": (C.c_int, [C.c_int, _pp]),
    "wpcg_ctx_destroy": (C.c_int, [_p]),
    "wpcg_ctx_stream": (C.c_int, [_p, _pp]),
    "wpcg_ctx_sync": (C.c_int, [_p]),
    "wpcg_dev_alloc": (C.c_int, [_p, C.c_size_t, _pp]),
    "wpcg_dev_free": (C.c_int, [_p, _p]),
    "wpcg_memcpy_h2d": (C.c_int, [_p, _p, _p, C.c_size_t]),
    "wpcg_memcpy_d2h": (C.c_int, [_p, _p, _p, C.c_size_t]),
    "wpcg_memcpy_d2d": (C.c_int, [_p, _p, _p, C.c_size_t]),
    "wpcg_event_create": (C.c_int, [_p, _pp]),
    "wpcg_event_destroy": (C.c_int, [_p]),
    "wpcg_event_record": (C.c_int, [_p, _p]),
    "wpcg_event_elapsed_ms": (C.c_int, [_p, _p, C.POINTER(C.c_float)]),
    "wpcg_artifact_open": (C.c_int, [C.c_char_p, C.c_int, _pp]),
    "wpcg_artifact_close": (C.c_int, [_p]),
    "wpcg_artifact_tensor": (C.c_int, [_p, C.c_char_p, _pp, _u64p]),
    "wpcg_artifact_tensor_count": (C.c_int, [_p, _u64p]),
    "wpcg_linear_create": (C.c_int, [_p, _p, C.c_char_p, _u64, _u64, _p, _pp]),
    "wpcg_linear_from_blocks": (C.c_int, [_p, C.c_int, _p, _u64, _u64, _u64, _p, _pp]),
    "wpcg_linear_destroy": (C.c_int, [_p]),
    "wpcg_linear_shape": (C.c_int, [_p, _u64p, _u64p]),
    "wpcg_linear_set_mode": (C.c_int, [_p, C.c_int]),
    "wpcg_linear_set_kslices": (C.c_int, [_p, C.c_int]),
    "wpcg_linear_set_fast_kernel": (C.c_int, [_p, C.c_int]),
    "wpcg_linear_kslices": (C.c_int, [_p, C.POINTER(C.c_int)]),
    "wpcg_plan_kslices": (C.c_int, [_u64, _u64, C.c_int, C.POINTER(C.c_int)]),
    "wpcg_linear_device_bytes": (C.c_int, [_p, _u64p]),
    "wpcg_linear_matvec": (C.c_int, [_p, _p, _p, _p]),
    "wpcg_linear_matvec_host": (C.c_int, [_p, _p, _p]),
    "wpcg_linear_gemm": (C.c_int, [_p, _p, C.c_int, C.c_uint32, _p, _p]),
    "wpcg_linear_gemm_host": (C.c_int, [_p, _p, C.c_int, C.c_uint32, _p]),
    "wpcg_linear_gemm_noalloc": (C.c_int, [_p, _p, C.c_int, C.c_uint32, _p, _p]),
    "wpcg_linear_set_gemm_kslices": (C.c_int, [_p, C.c_int]),
    "wpcg_linear_gemm_kslices": (C.c_int, [_p, _p, _p]),
    "wpcg_linear_embed": (C.c_int, [_p, C.c_uint32, _p, _p]),
    "wpcg_linear_embed_host": (C.c_int, [_p, C.c_uint32, _p]),
    "wpcg_linear_dequant": (C.c_int, [_p, C.c_int, _p, _p]),
    "wpcg_linear_clone": (C.c_int, [_p, _pp]),
    "wpcg_linear_matvec_multi": (C.c_int, [C.c_int, _pp, _pp, _pp, _p]),
    "wpcg_encode": (C.c_int, [C.c_int, _p, _u64, _p]),
    "wpcg_model_create": (C.c_int, [_p, C.c_int, _p, _pp]),
    "wpcg_model_destroy": (C.c_int, [_p]),
    "wpcg_model_set_tensor": (C.c_int, [_p, C.c_char_p, _p, _u64]),
    "wpcg_model_load_artifact": (C.c_int, [_p, _p]),
    "wpcg_model_load_safetensors": (C.c_int, [_p, _p]),
    "wpcg_safetensors_open": (C.c_int, [C.c_char_p, _pp]),
    "wpcg_safetensors_open_file": (C.c_int, [C.c_char_p, _pp]),
    "wpcg_safetensors_close": (C.c_int, [_p]),
    "wpcg_safetensors_tensor_count": (C.c_int, [_p, _u64p]),
    "wpcg_safetensors_name": (C.c_int, [_p, _u64, C.POINTER(C.c_char_p)]),
    "wpcg_safetensors_shape": (C.c_int, [_p, C.c_char_p, C.POINTER(C.c_uint32), _u64p, C.c_uint32]),
    "wpcg_safetensors_dtype": (C.c_int, [_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "wpcg_safetensors_read_f32": (C.c_int, [_p, C.c_char_p, _p, _u64]),
    "wpcg_config_parse": (C.c_int, [C.c_char_p, C.c_uint32, _p]),
    "wpcg_config_load": (C.c_int, [C.c_char_p, C.c_uint32, _p]),
    "wpcg_model_set_mode": (C.c_int, [_p, C.c_int]),
    "wpcg_model_reset": (C.c_int, [_p]),
    "wpcg_model_set_graphs": (C.c_int, [_p, C.c_int]),
    "wpcg_model_position": (C.c_int, [_p, C.POINTER(C.c_uint32)]),
    "wpcg_model_forward_token": (C.c_int, [_p, C.c_uint32, _p, C.POINTER(C.c_uint32)]),
    "wpcg_model_generate": (C.c_int, [_p, _p, C.c_uint32, C.c_uint32, _p, C.POINTER(C.c_float)]),
    "wpcg_model_prefill": (C.c_int, [_p, _p, C.c_uint32, _p, C.POINTER(C.c_uint32)]),
    "wpcg_model_set_prefill": (C.c_int, [_p, C.c_int]),
    "wpcg_model_verify": (C.c_int, [_p, _p, C.c_uint32, _p, _p]),
    "wpcg_model_set_position": (C.c_int, [_p, C.c_uint32]),
    "wpcg_model_debug_read": (C.c_int, [_p, C.c_int, _p, _u64]),
    "wpcg_rms_norm": (C.c_int, [_p, _p, _p, C.c_uint32, C.c_float, _p, C.c_int, _p]),
    "wpcg_dense_create": (C.c_int, [_p, _p, _u64, _u64, _p, _pp]),
    "wpcg_dense_destroy": (C.c_int, [_p]),
    "wpcg_dense_set_mode": (C.c_int, [_p, C.c_int]),
    "wpcg_dense_matvec": (C.c_int, [_p, _p, _p, _p]),
    "wpcg_softmax": (C.c_int, [_p, _p, C.c_uint32, _p]),
    "wpcg_route": (C.c_int, [_p, _p, C.c_uint32, C.c_uint32, C.c_int, _p, _p, _p]),
    "wpcg_silu_mul": (C.c_int, [_p, _p, _p, _p, _u64, _p]),
    "wpcg_moe_create": (C.c_int, [_p, C.c_int, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                  C.c_int, _pp]),
    "wpcg_moe_destroy": (C.c_int, [_p]),
    "wpcg_moe_set_router": (C.c_int, [_p, _p]),
    "wpcg_moe_set_expert": (C.c_int, [_p, C.c_uint32, _p, _p, _p]),
    "wpcg_moe_load_experts": (C.c_int, [_p, _p, C.c_uint32]),
    "wpcg_moe_set_mode": (C.c_int, [_p, C.c_int]),
    "wpcg_moe_forward": (C.c_int, [_p, _p, _p, _p, _p, _p]),
    "wpcg_graph_begin": (C.c_int, [_p]),
    "wpcg_graph_end": (C.c_int, [_p, _pp]),
    "wpcg_graph_launch": (C.c_int, [_p, _p]),
    "wpcg_graph_destroy": (C.c_int, [_p]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def declared_symbols(header: str = HEADER) -> list[str]:
    """Function names declared in include/wpcg.h."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wpcg_[a-z0-9_]+)\s*\(", text)))


def last_error() -> str:
    return (lib.wpcg_last_error_string() or b"").decode()


def check(rc: int) -> None:
    if rc != OK:
        raise WpcgError(rc, last_error())


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def matvec_multi(lins, xs, ys, stream=None):
    """ys[i] = lins[i] @ xs[i] for device buffers, grouped into shared launches."""
    n = len(lins)
    arr = (C.c_void_p * n)
    check(lib.wpcg_linear_matvec_multi(n, arr(*[l.h for l in lins]), arr(*[x.ptr for x in xs]),
                                       arr(*[y.ptr for y in ys]), stream))


def plan_kslices(out_f: int, in_f: int, requested: int = 0) -> int:
    k = C.c_int()
    check(lib.wpcg_plan_kslices(out_f, in_f, requested, C.byref(k)))
    return k.value


def device_count() -> int:
    n = C.c_int(0)
    rc = lib.wpcg_device_count(C.byref(n))
    return n.value if rc == OK else 0


# Every wrapper of a native handle registers itself here, in creation order.
# release_all() releases the live ones newest first, so each handle goes
# before anything it was made from (a linear before its context, a graph
# before the buffers it was captured over); an atexit hook runs it, so a
# process that leaves normally has destroyed every stream, graph, event and
# device buffer of this library before the ROCm runtime's own exit-time
# teardown begins.
_tracked = []
_gpu_used = False
# Processes that used the GPU leave through the interpreter's normal exit
# after release_all() (NORMAL_EXIT). WPCG_HARD_EXIT=1 ends them with os._exit
# after release_all() instead, skipping the runtime's exit-time teardown:
# that teardown once aborted (std::bad_variant_access thrown from a runtime
# library) when handles were left to Python's finalizers at shutdown.
NORMAL_EXIT = os.environ.get("WPCG_HARD_EXIT", "") != "1"


def _track(obj):
    _tracked.append(weakref.ref(obj))
    if len(_tracked) > 4096 and len(_tracked) % 4096 == 0:  # drop dead references now and then
        _tracked[:] = [r for r in _tracked if r() is not None]


def gpu_used() -> bool:
    return _gpu_used


def release_all() -> int:
    """Releases every native handle still alive, newest first; contexts are
    synchronized before they are destroyed. Returns the number of errors."""
    errors = 0
    for r in reversed(_tracked):
        o = r()
        if o is None:
            continue
        try:
            if isinstance(o, Context) and o.h:
                o.sync()
            o._release()
        except Exception as e:  # report, and keep releasing
            print(f"wpcg: release error: {e}", file=sys.stderr)
            errors += 1
    _tracked.clear()
    return errors


atexit.register(release_all)


def hard_exit(code: int = 0):
    """release_all(), flush, then os._exit(code)."""
    if release_all():
        code = code or 1
    sys.stdout.flush()
    sys.stderr.flush()
    os._exit(code)


def finish(code: int = 0) -> int:
    """The end of a process that used the GPU: release_all(), then either
    return `code` for a normal exit (NORMAL_EXIT) or leave through
    hard_exit."""
    if not NORMAL_EXIT:
        hard_exit(code)
    if release_all():
        code = code or 1
    return code


# ------------------------------------------------------------------ device
class Context:
    """One GPU and its default stream."""

    def __init__(self, device: int = 0):
        global _gpu_used
        h = C.c_void_p()
        check(lib.wpcg_ctx_create(device, C.byref(h)))
        _gpu_used = True
        self.h = h
        _track(self)
        s = C.c_void_p()
        check(lib.wpcg_ctx_stream(self.h, C.byref(s)))
        self.stream = s

    def sync(self):
        check(lib.wpcg_ctx_sync(self.h))

    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes)
        b.write(arr)
        return b

    def event(self) -> "Event":
        return Event(self)

    def capture(self, fn) -> "Graph":
        """Records the device calls fn() makes on the context stream."""
        check(lib.wpcg_graph_begin(self.h))
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = lib.wpcg_graph_end(self.h, C.byref(g))
        check(rc)
        return Graph(self, g)

    def close(self):
        if self.h:
            lib.wpcg_ctx_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    def __init__(self, ctx: Context, nbytes: int):
        self.ctx, self.nbytes = ctx, int(nbytes)
        p = C.c_void_p()
        check(lib.wpcg_dev_alloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p
        _track(self)

    def write(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib.wpcg_memcpy_h2d(self.ctx.h, self.ptr, _np_ptr(arr), arr.nbytes))

    def read(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        check(lib.wpcg_memcpy_d2h(self.ctx.h, _np_ptr(out), self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib.wpcg_dev_free(self.ctx.h, self.ptr)
            self.ptr = None

    def _release(self):
        if self.ctx.h:
            self.free()

    def __del__(self):
        try:
            if self.ctx.h:
                self.free()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        h = C.c_void_p()
        check(lib.wpcg_event_create(ctx.h, C.byref(h)))
        self.h = h
        _track(self)

    def record(self, stream=None):
        check(lib.wpcg_event_record(self.h, stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib.wpcg_event_elapsed_ms(self.h, end.h, C.byref(ms)))
        return ms.value

    def _release(self):
        if self.h:
            lib.wpcg_event_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: Context, h):
        self.ctx, self.h = ctx, h
        _track(self)

    def launch(self, stream=None):
        check(lib.wpcg_graph_launch(self.h, stream))

    def _release(self):
        if self.h:
            lib.wpcg_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


# ------------------------------------------------------------------ artifact
class WpcModelData:
    """model_v{3,4}.meta + mmap of model_v{3,4}.wpc (WpcModelDataV4::open)."""

    scheme = SCHEME_V4

    def __init__(self, h, scheme):
        self.h, self.scheme = h, scheme
        _track(self)

    @classmethod
    def open(cls, wpc_dir: str, scheme: int | None = None):
        scheme = cls.scheme if scheme is None else scheme
        h = C.c_void_p()
        check(lib.wpcg_artifact_open(os.fsencode(wpc_dir), scheme, C.byref(h)))
        return cls(h, scheme)

    def tensor_bytes(self, name: str) -> np.ndarray:
        p, n = C.c_void_p(), C.c_uint64()
        check(lib.wpcg_artifact_tensor(self.h, name.encode(), C.byref(p), C.byref(n)))
        if n.value == 0:
            return np.zeros(0, np.uint8)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), (n.value,)).copy()

    def tensor_count(self) -> int:
        n = C.c_uint64()
        check(lib.wpcg_artifact_tensor_count(self.h, C.byref(n)))
        return n.value

    def close(self):
        if self.h:
            lib.wpcg_artifact_close(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WpcModelDataV4(WpcModelData):
    scheme = SCHEME_V4


class WpcModelDataV3(WpcModelData):
    scheme = SCHEME_V3


# ------------------------------------------------------------------ linear
class WpcLinear:
    """A quantized matrix resident on the GPU (trait Linear)."""

    def __init__(self, ctx: Context, h):
        self.ctx, self.h = ctx, h
        _track(self)
        o, i = C.c_uint64(), C.c_uint64()
        check(lib.wpcg_linear_shape(h, C.byref(o), C.byref(i)))
        self._out, self._in = o.value, i.value

    @classmethod
    def from_artifact(cls, ctx: Context, data: WpcModelData, name: str, out_f: int, in_f: int,
                      bias=None):
        h = C.c_void_p()
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        check(lib.wpcg_linear_create(ctx.h if ctx else None, data.h, name.encode(), out_f, in_f,
                                     None if b is None else _np_ptr(b), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_blocks(cls, ctx: Context, scheme: int, blocks: np.ndarray, out_f: int, in_f: int,
                    bias=None):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        check(lib.wpcg_linear_from_blocks(ctx.h if ctx else None, scheme, _np_ptr(blocks),
                                          blocks.nbytes, out_f, in_f,
                                          None if b is None else _np_ptr(b), C.byref(h)))
        return cls(ctx, h)

    def in_features(self) -> int:
        return self._in

    def out_features(self) -> int:
        return self._out

    def set_mode(self, mode: int):
        check(lib.wpcg_linear_set_mode(self.h, mode))
        return self

    def set_kslices(self, k: int):
        check(lib.wpcg_linear_set_kslices(self.h, k))
        return self

    def set_fast_kernel(self, kernel: int):
        """FAST_KERNEL_MFMA (default) or FAST_KERNEL_VALU for plain GEMVs."""
        check(lib.wpcg_linear_set_fast_kernel(self.h, kernel))
        return self

    def kslices(self) -> int:
        k = C.c_int()
        check(lib.wpcg_linear_kslices(self.h, C.byref(k)))
        return k.value

    def device_bytes(self) -> int:
        n = C.c_uint64()
        check(lib.wpcg_linear_device_bytes(self.h, C.byref(n)))
        return n.value

    def matvec(self, x) -> np.ndarray:
        """Linear::matvec with host arrays (synchronous)."""
        x = np.ascontiguousarray(x, np.float32)
        assert x.size == self._in
        y = np.empty(self._out, np.float32)
        check(lib.wpcg_linear_matvec_host(self.h, _np_ptr(x), _np_ptr(y)))
        return y

    def matvec_dev(self, x: DeviceBuffer, y: DeviceBuffer, stream=None):
        check(lib.wpcg_linear_matvec(self.h, x.ptr, y.ptr, stream))

    def gemm(self, X, dtype: int = DTYPE_F32) -> np.ndarray:
        """Y = X W^T (+ bias) for a batch X of shape (M, in_features): fp32
        values (DTYPE_F32 rounds them to bf16, DTYPE_F32_SPLIT carries them
        as two bf16 terms), or bf16 bit patterns (uint16) with DTYPE_BF16."""
        X = np.ascontiguousarray(X, np.uint16 if dtype == DTYPE_BF16 else np.float32)
        assert X.ndim == 2 and X.shape[1] == self._in
        Y = np.empty((X.shape[0], self._out), np.float32)
        check(lib.wpcg_linear_gemm_host(self.h, _np_ptr(X), dtype, X.shape[0], _np_ptr(Y)))
        return Y

    def gemm_dev(self, X: DeviceBuffer, M: int, Y: DeviceBuffer, dtype: int = DTYPE_F32, stream=None):
        check(lib.wpcg_linear_gemm(self.h, X.ptr, dtype, M, Y.ptr, stream))

    def set_gemm_kslices(self, k: int):
        check(lib.wpcg_linear_set_gemm_kslices(self.h, k))
        return self

    def gemm_kslices(self) -> tuple[int, int]:
        """(K-slices for M <= 16, K-slices for M > 16)."""
        a, b = C.c_int(), C.c_int()
        check(lib.wpcg_linear_gemm_kslices(self.h, C.byref(a), C.byref(b)))
        return a.value, b.value

    def embed(self, token: int) -> np.ndarray:
        out = np.empty(self._in, np.float32)
        check(lib.wpcg_linear_embed_host(self.h, token, _np_ptr(out)))
        return out

    def logits(self, x) -> np.ndarray:
        return self.matvec(x)

    def clone(self) -> "WpcLinear":
        h = C.c_void_p()
        check(lib.wpcg_linear_clone(self.h, C.byref(h)))
        return WpcLinear(self.ctx, h)

    def dequant(self, rounding: int) -> np.ndarray:
        buf = self.ctx.alloc(self._out * self._in * 4)
        check(lib.wpcg_linear_dequant(self.h, rounding, buf.ptr, None))
        self.ctx.sync()
        out = buf.read(np.float32, self._out * self._in).reshape(self._out, self._in)
        buf.free()
        return out

    def close(self):
        if self.h:
            lib.wpcg_linear_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WpcLinearV4(WpcLinear):
    def __init__(self, ctx, data_or_h, name=None, out_f=None, in_f=None, bias=None):
        if name is None:
            super().__init__(ctx, data_or_h)
        else:
            tmp = WpcLinear.from_artifact(ctx, data_or_h, name, out_f, in_f, bias)
            super().__init__(ctx, tmp.h)
            tmp.h = None


class WpcLinearV3(WpcLinearV4):
    pass


WpcEmbeddingV4 = WpcLinearV4
WpcEmbeddingV3 = WpcLinearV3


# ------------------------------------------------------------------ MoE pieces
class DenseLinear:
    """fp32 dense matrix on the GPU (DenseLinear, weights.rs:35-79; the
    Qwen3-MoE router)."""

    def __init__(self, ctx: Context, w, bias=None):
        w = np.ascontiguousarray(w, np.float32)
        self.ctx, (self._out, self._in) = ctx, w.shape
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        h = C.c_void_p()
        check(lib.wpcg_dense_create(ctx.h if ctx else None, _np_ptr(w), self._out, self._in,
                                    None if b is None else _np_ptr(b), C.byref(h)))
        self.h = h
        _track(self)

    def in_features(self) -> int:
        return self._in

    def out_features(self) -> int:
        return self._out

    def set_mode(self, mode: int):
        check(lib.wpcg_dense_set_mode(self.h, mode))
        return self

    def matvec_dev(self, x: DeviceBuffer, y: DeviceBuffer, stream=None):
        check(lib.wpcg_dense_matvec(self.h, x.ptr, y.ptr, stream))

    def matvec(self, x) -> np.ndarray:
        xb = self.ctx.upload(np.ascontiguousarray(x, np.float32))
        yb = self.ctx.alloc(4 * self._out)
        self.matvec_dev(xb, yb)
        self.ctx.sync()
        return yb.read(np.float32, self._out)

    def close(self):
        if self.h:
            lib.wpcg_dense_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def softmax(ctx: Context, x) -> np.ndarray:
    """softmax_inplace (norm.rs:28-43) on the GPU, returned to the host."""
    x = np.ascontiguousarray(x, np.float32)
    b = ctx.upload(x)
    check(lib.wpcg_softmax(ctx.h, b.ptr, x.size, None))
    ctx.sync()
    return b.read(np.float32, x.size)


def rms_norm(ctx: Context, x, w, eps: float, mode: int = MODE_EXACT) -> np.ndarray:
    """rms_norm (norm.rs:4-13) on the GPU, returned to the host."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    xb, wb, ob = ctx.upload(x), ctx.upload(w), ctx.alloc(4 * x.size)
    check(lib.wpcg_rms_norm(ctx.h, xb.ptr, wb.ptr, x.size, eps, ob.ptr, mode, None))
    ctx.sync()
    return ob.read(np.float32, x.size)


def route(ctx: Context, probs, top_k: int, norm_topk: bool = True):
    """Qwen3MoeModel::route (qwen3_moe_model.rs:376-402) on the GPU:
    (ids int32[top_k], weights float32[top_k])."""
    p = np.ascontiguousarray(probs, np.float32)
    b, ib, wb = ctx.upload(p), ctx.alloc(4 * top_k), ctx.alloc(4 * top_k)
    check(lib.wpcg_route(ctx.h, b.ptr, p.size, top_k, int(bool(norm_topk)), ib.ptr, wb.ptr, None))
    ctx.sync()
    return ib.read(np.int32, top_k), wb.read(np.float32, top_k)


def silu_mul(ctx: Context, g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    gb, ub, ob = ctx.upload(g), ctx.upload(u), ctx.alloc(4 * g.size)
    check(lib.wpcg_silu_mul(ctx.h, gb.ptr, ub.ptr, ob.ptr, g.size, None))
    ctx.sync()
    return ob.read(np.float32, g.size)


class MoeLayer:
    """The routed-expert MLP of one Qwen3-MoE layer, resident on the GPU
    (qwen3_moe_model.rs:500-530)."""

    def __init__(self, ctx: Context, scheme: int, n_exp: int, hidden: int, inter: int,
                 top_k: int, norm_topk: bool = True):
        self.ctx = ctx
        self.n_exp, self.hidden, self.inter, self.top_k = n_exp, hidden, inter, top_k
        h = C.c_void_p()
        check(lib.wpcg_moe_create(ctx.h if ctx else None, scheme, n_exp, hidden, inter, top_k,
                                  int(bool(norm_topk)), C.byref(h)))
        self.h = h
        _track(self)

    def set_router(self, w):
        w = np.ascontiguousarray(w, np.float32)
        assert w.shape == (self.n_exp, self.hidden)
        check(lib.wpcg_moe_set_router(self.h, _np_ptr(w)))
        return self

    def set_expert(self, e: int, gate, up, down):
        g, u, d = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
        check(lib.wpcg_moe_set_expert(self.h, e, _np_ptr(g), _np_ptr(u), _np_ptr(d)))
        return self

    def load_experts(self, data: "WpcModelData", layer: int):
        check(lib.wpcg_moe_load_experts(self.h, data.h, layer))
        return self

    def set_mode(self, mode: int):
        check(lib.wpcg_moe_set_mode(self.h, mode))
        return self

    def forward_dev(self, x: DeviceBuffer, out: DeviceBuffer, ids=None, weights=None, stream=None):
        check(lib.wpcg_moe_forward(self.h, x.ptr, out.ptr, ids.ptr if ids else None,
                                   weights.ptr if weights else None, stream))

    def forward(self, x):
        """(out float32[hidden], ids int32[top_k], weights float32[top_k])"""
        xb = self.ctx.upload(np.ascontiguousarray(x, np.float32))
        ob, ib, wb = self.ctx.alloc(4 * self.hidden), self.ctx.alloc(4 * self.top_k), self.ctx.alloc(4 * self.top_k)
        self.forward_dev(xb, ob, ib, wb)
        self.ctx.sync()
        return ob.read(np.float32, self.hidden), ib.read(np.int32, self.top_k), wb.read(np.float32, self.top_k)

    def close(self):
        if self.h:
            lib.wpcg_moe_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------ encoder
def encode(scheme: int, w) -> np.ndarray:
    """encode_tensor_v{4,3} (quant_encoder.rs): fp32 values (a multiple of
    128) to reference blocks, on the host."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    out = np.empty(w.size // 128 * (68 if scheme == SCHEME_V4 else 100), np.uint8)
    check(lib.wpcg_encode(scheme, _np_ptr(w), w.size, _np_ptr(out)))
    return out


# ------------------------------------------------------------------ decode
class ModelConfig(C.Structure):
    """wpcg_model_config (include/wpcg.h)."""
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("inter", C.c_uint32),
                ("vocab", C.c_uint32), ("n_experts", C.c_uint32), ("top_k", C.c_uint32),
                ("moe_inter", C.c_uint32), ("norm_topk", C.c_int32), ("tied", C.c_int32),
                ("max_pos", C.c_uint32), ("eps", C.c_float), ("rope_theta", C.c_double)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


def config_from_json_str(text: str, max_pos: int) -> ModelConfig:
    """Config::from_json_str (wpc-runtime/src/config.rs:85-88) with head_dim
    (config.rs:59-62) and, for Qwen3-MoE, moe_dims
    (qwen3_moe_model.rs:121-135) resolved; max_pos is the KV-cache length."""
    cfg = ModelConfig()
    check(lib.wpcg_config_parse(text.encode(), max_pos, C.byref(cfg)))
    return cfg


def config_load(path, max_pos: int) -> ModelConfig:
    """Config::load (config.rs:90-93)."""
    cfg = ModelConfig()
    check(lib.wpcg_config_load(os.fsencode(path), max_pos, C.byref(cfg)))
    return cfg


class ShardedSafetensors:
    """A checkpoint directory: model.safetensors, or the shards its
    model.safetensors.index.json names (ShardedSafetensors,
    wpc-runtime/src/weights.rs:180-264). Host memory only."""

    def __init__(self, handle):
        self.h = handle
        _track(self)

    @classmethod
    def open(cls, model_dir) -> "ShardedSafetensors":
        h = C.c_void_p()
        check(lib.wpcg_safetensors_open(os.fsencode(model_dir), C.byref(h)))
        return cls(h)

    def names(self) -> list[str]:
        n = C.c_uint64()
        check(lib.wpcg_safetensors_tensor_count(self.h, C.byref(n)))
        out = []
        for i in range(n.value):
            p = C.c_char_p()
            check(lib.wpcg_safetensors_name(self.h, i, C.byref(p)))
            out.append(p.value.decode())
        return out

    def shape(self, name: str) -> list[int]:
        nd = C.c_uint32()
        dims = (C.c_uint64 * 16)()
        check(lib.wpcg_safetensors_shape(self.h, name.encode(), C.byref(nd), dims, 16))
        return [dims[i] for i in range(nd.value)]

    def dtype(self, name: str) -> str:
        p = C.c_char_p()
        check(lib.wpcg_safetensors_dtype(self.h, name.encode(), C.byref(p)))
        return p.value.decode()

    def read_f32(self, name: str) -> np.ndarray:
        """The tensor widened to float32, flat row-major."""
        n = int(np.prod(self.shape(name), dtype=np.uint64))
        out = np.empty(n, np.float32)
        check(lib.wpcg_safetensors_read_f32(self.h, name.encode(), _np_ptr(out), n))
        return out

    def close(self):
        if self.h:
            lib.wpcg_safetensors_close(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SafetensorsFile(ShardedSafetensors):
    """One .safetensors file (SafetensorsFile, weights.rs:125-178)."""

    @classmethod
    def open(cls, path) -> "SafetensorsFile":
        h = C.c_void_p()
        check(lib.wpcg_safetensors_open_file(os.fsencode(path), C.byref(h)))
        return cls(h)


class Model:
    """Dense Qwen3 / Qwen3-MoE decoder resident on the GPU
    (Model::forward_token, model.rs:419-547; qwen3_moe_model.rs:406-542)."""

    def __init__(self, ctx: Context, scheme: int, cfg: ModelConfig):
        self.ctx, self.scheme, self.cfg = ctx, scheme, cfg
        h = C.c_void_p()
        check(lib.wpcg_model_create(ctx.h if ctx else None, scheme, C.byref(cfg), C.byref(h)))
        self.h = h
        _track(self)

    def set_tensor(self, name: str, data: np.ndarray):
        data = np.ascontiguousarray(data)
        check(lib.wpcg_model_set_tensor(self.h, name.encode(), _np_ptr(data), data.nbytes))
        return self

    def load_artifact(self, data: "WpcModelData"):
        check(lib.wpcg_model_load_artifact(self.h, data.h))
        return self

    def load_safetensors(self, st: ShardedSafetensors):
        """Norms and routers from the dense checkpoint, as load_wpc_v4 reads
        them (qwen3_moe_model.rs:140-196, 327-365; qwen3_model.rs:40-90)."""
        check(lib.wpcg_model_load_safetensors(self.h, st.h))
        return self

    @classmethod
    def load_wpc(cls, ctx: Context, scheme: int, model_dir, wpc_dir, max_pos: int) -> "Model":
        """load_wpc_v4 / load_wpc_v3 (qwen3_moe_model.rs:327-365,
        qwen3_model.rs:187-206): config.json and the fp32 tensors from
        model_dir, every quantized matrix from the artifact in wpc_dir."""
        cfg = config_load(os.path.join(os.fsdecode(model_dir), "config.json"), max_pos)
        m = cls(ctx, scheme, cfg)
        st = ShardedSafetensors.open(model_dir)
        try:
            m.load_safetensors(st)
        finally:
            st.close()
        data = WpcModelData.open(wpc_dir, scheme)
        try:
            m.load_artifact(data)
        finally:
            data.close()
        return m

    def set_mode(self, mode: int):
        check(lib.wpcg_model_set_mode(self.h, mode))
        return self

    def reset(self):
        check(lib.wpcg_model_reset(self.h))
        return self

    def set_graphs(self, enabled: bool):
        check(lib.wpcg_model_set_graphs(self.h, int(bool(enabled))))
        return self

    def position(self) -> int:
        p = C.c_uint32()
        check(lib.wpcg_model_position(self.h, C.byref(p)))
        return p.value

    def forward_token(self, token: int, want_logits: bool = True):
        """(logits float32[vocab] or None, argmax)"""
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        a = C.c_uint32()
        check(lib.wpcg_model_forward_token(self.h, token, None if logits is None else _np_ptr(logits),
                                           C.byref(a)))
        return logits, a.value

    def prefill(self, tokens, want_logits: bool = True):
        """The tokens at the next positions as forward_token would run them
        one by one (FAST: batched): (logits of the last or None, argmax)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        a = C.c_uint32()
        check(lib.wpcg_model_prefill(self.h, _np_ptr(t), t.size, None if logits is None else _np_ptr(logits),
                                     C.byref(a)))
        return logits, a.value

    def verify(self, tokens, want_logits: bool = False):
        """(argmax after each token uint32[n], logits [n][vocab] or None)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        ids = np.empty(t.size, np.uint32)
        logits = np.empty((t.size, self.cfg.vocab), np.float32) if want_logits else None
        check(lib.wpcg_model_verify(self.h, _np_ptr(t), t.size, _np_ptr(ids),
                                    None if logits is None else _np_ptr(logits)))
        return ids, logits

    def set_position(self, pos: int):
        check(lib.wpcg_model_set_position(self.h, pos))
        return self

    def set_prefill(self, enabled: bool):
        check(lib.wpcg_model_set_prefill(self.h, int(bool(enabled))))
        return self

    def generate(self, prompt, n_new: int):
        """(new token ids uint32[n_new], ms of the n_new-1 steps after the prompt)"""
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_new, np.uint32)
        ms = C.c_float()
        check(lib.wpcg_model_generate(self.h, _np_ptr(p), p.size, n_new, _np_ptr(out), C.byref(ms)))
        return out, ms.value

    def debug_read(self, which: int, n: int) -> np.ndarray:
        """A device buffer of the last step (see wpcg_model_debug_read)."""
        out = np.empty(n, np.float32)
        check(lib.wpcg_model_debug_read(self.h, which, _np_ptr(out), n))
        return out

    def close(self):
        if self.h:
            lib.wpcg_model_destroy(self.h)
            self.h = None

    _release = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
