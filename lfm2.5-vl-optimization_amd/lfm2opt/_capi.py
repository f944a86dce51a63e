"""ctypes binding of liblfm2q.so (the C ABI declared in include/lfm2q.h).

torch is imported before the library is opened: the shared object links against libamdhip64.so.7 by SONAME, and
loading it after torch makes it use the HIP runtime torch already loaded, so the hipStream_t handles torch hands out
are valid in the library. There is no fallback: if the library is missing, every op raises.
"""

import ctypes
import pathlib

import torch  # noqa: F401  (must precede the dlopen below, see module docstring)

LIB_PATH = pathlib.Path(__file__).resolve().parent.parent / "lib" / "liblfm2q.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


class GemvOp(ctypes.Structure):
    """lfm2q_gemv_op: one GEMV of a chain (include/lfm2q.h)."""
    _fields_ = [("W", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("N", ctypes.c_int32), ("K", ctypes.c_int32), ("epi", ctypes.c_int32), ("reserved", ctypes.c_int32)]


# entry points that return something other than an int status
RESTYPES = {"lfm2q_gemv_chain_workspace_bytes": ctypes.c_size_t, "lfm2q_gemm_workspace_bytes": ctypes.c_size_t}

# name -> argument types (every entry point returns an int status unless listed in RESTYPES)
SIGNATURES = {
    "lfm2q_gemv_w8": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemv_bf16": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemv_swiglu": [_I, _P, _P, _P, _P, _I, _I, _I, _P],
    "lfm2q_gemv_residual": [_I, _P, _P, _P, _P, _I, _I, _I, _P],
    "lfm2q_gemv_rmsnorm": [_I, _I, _P, _P, _P, _P, _F, _P, _I, _I, _P],
    "lfm2q_gemv_w4": [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "lfm2q_silu_mul": [_P, _P, _I, _I, _P],
    "lfm2q_quant_rows": [_P, _P, _P, _I, _I, _P],
    "lfm2q_quant_groups": [_P, _P, _P, _I, _I, _P],
    "lfm2q_add_rmsnorm_q": [_P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _P],
    "lfm2q_add_layernorm_q": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _P],
    "lfm2q_silu_mul_q": [_P, _P, _P, _P, _I, _I, _I, _P],
    "lfm2q_gemm_i8": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemm_i8_ex": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "lfm2q_gemm_workspace_bytes": [],
    "lfm2q_gemm_i8_grouped": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemm_i8_bf16a": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemm_i8_fq": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "lfm2q_gemm_i8_q": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemm_w8": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "lfm2q_gemm_w8_ex": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "lfm2q_gemm_i8_i32": [_P, _P, _P, _I, _I, _I, _P],
    "lfm2q_gemv_chain": [_P, _P, _I, _P, ctypes.c_size_t, _P],
    "lfm2q_gemv_chain_noalloc": [_P, _P, _I, _P, _P],
    "lfm2q_gemv_chain_workspace_bytes": [],
    "lfm2q_set_tuning": [ctypes.c_char_p, ctypes.c_char_p],
    "lfm2q_get_tuning": [ctypes.c_char_p, ctypes.POINTER(_I), ctypes.POINTER(_I)],
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"liblfm2q.so is not built ({LIB_PATH}); build it with "
                               f"`make -C lfm2.5-vl-optimization_amd/csrc` or __graft_entry__.build()")
        L = ctypes.CDLL(str(LIB_PATH))
        L.lfm2q_last_error.restype = ctypes.c_char_p
        L.lfm2q_last_error.argtypes = []
        L.lfm2q_version.restype = ctypes.c_char_p
        L.lfm2q_version.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def call(name, *args):
    """Call entry point `name`; a non-zero status becomes RuntimeError with the library's message."""
    st = getattr(lib(), name)(*args)
    if st != 0:
        raise RuntimeError(lib().lfm2q_last_error().decode())


def set_tuning(name, value=None):
    """Force a launch configuration (lfm2q_set_tuning): value "a,b,..." or an int, None = automatic."""
    call("lfm2q_set_tuning", name.encode(), None if value is None else str(value).encode())


def get_tuning(name):
    """The knob's values as a tuple (empty = automatic)."""
    vals, n = (_I * 4)(), _I(0)
    call("lfm2q_get_tuning", name.encode(), vals, ctypes.byref(n))
    return tuple(vals[: n.value])


def stream(t):
    """Raw hipStream_t of torch's current stream on t's device (the reference launches on the same stream)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


_workspaces = {}


def _ws_key(device, stream):
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    s = torch.cuda.current_stream(device) if stream is None else stream
    return device, (device.index, s.cuda_stream)


def prepare_workspace(device=None, stream=None):
    """Create (and zero-fill, by a fill kernel on that stream) the GEMM workspace of `stream` (default: torch's
    current stream) on `device`, if it does not exist yet, and return it. Call it on a capture stream before
    capturing: the fill must not be recorded into a graph."""
    device, key = _ws_key(device, stream)
    w = _workspaces.get(key)
    if w is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("lfm2q: the GEMM workspace of this stream does not exist yet and the stream is being "
                               "captured; call lfm2opt.kernels.prepare_workspace() on the capture stream before the "
                               "capture (its zero fill must stay out of the graph)")
        s = torch.cuda.current_stream(device) if stream is None else stream
        with torch.cuda.stream(s):
            w = torch.zeros(lib().lfm2q_gemm_workspace_bytes(), dtype=torch.uint8, device=device)
        _workspaces[key] = w
    return w


def release_workspace(device=None, stream=None):
    """Drop the GEMM workspace of `stream` on `device` (its memory returns to torch's allocator once no other
    reference remains). Only when no call on that stream is in flight and no captured graph that used it will be
    replayed again: such a graph keeps the workspace's address. Returns whether there was one."""
    _, key = _ws_key(device, stream)
    return _workspaces.pop(key, None) is not None


def workspace(t):
    """The GEMM workspace of torch's current stream on t's device: lfm2q_gemm_workspace_bytes() of device memory
    (arrival counters for the K split across workgroups, then the partial tiles), zero-filled when first used and
    kept until release_workspace(). Calls on one stream are ordered, so they share it; another stream gets its own
    (so a caller that makes a stream per request should release it afterwards). A graph captured on a stream uses
    that stream's workspace, so graphs captured on one stream must not be replayed concurrently with each other.
    Inside a capture the stream's workspace must already exist (an eager call on that stream, or
    prepare_workspace()): otherwise this raises, since a zero fill recorded into one graph would leave the counters
    undefined for every later graph and eager call that shares the buffer."""
    return prepare_workspace(t.device)
