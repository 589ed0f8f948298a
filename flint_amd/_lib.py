"""ctypes binding of libflint_amd.so (the C ABI declared in include/flint_amd.h).

The product path calls the HIP library only; there is no CPU or torch fallback. If the
library is missing, every entry point raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FLINT_AMD_LIB", os.path.join(HERE, "libflint_amd.so"))

FL_OK = 0
ERRORS = {
    -1: "FL_E_ARG (bad argument / unsupported shape)",
    -2: "FL_E_POS (position beyond max_seq or rope table)",
    -3: "FL_E_M (verify width out of range)",
    -4: "FL_E_LAUNCH (HIP launch failed)",
    -5: "FL_E_HIP (HIP runtime error)",
    -6: "FL_E_TIMEOUT (an inter-workgroup wait hit its time limit)",
}
MAX_VERIFY = 32
HEAD_DIM = 64
GROUP = 128

# every symbol include/flint_amd.h declares
EXPORTS = [
    "fl_version", "fl_device_info", "fl_quantize_int4", "fl_dequant_int4", "fl_dequant_int4_mx", "fl_gemv_int4",
    "fl_gemm_int4", "fl_state_create", "fl_state_destroy", "fl_state_reset", "fl_state_check",
    "fl_state_profile", "fl_state_buffers", "fl_state_set_wait_limit",
    "fl_state_force_timeout",
    "fl_decode_step", "fl_decode_sample", "fl_decode_hidden", "fl_verify", "fl_kv_move", "fl_sample",
    "fl_sample_noalloc", "fl_probe_handoff", "fl_tile_int4", "fl_dequant_int4_tiled", "fl_gemv_int4_tiled",
    "fl_probe_dequant",
]


class FlError(RuntimeError):
    def __init__(self, fn, code):
        super().__init__(f"{fn} failed: {ERRORS.get(code, code)}")
        self.code = code


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int32), ("dim", ctypes.c_int32), ("n_head", ctypes.c_int32),
        ("n_kv_head", ctypes.c_int32), ("inter", ctypes.c_int32), ("vocab", ctypes.c_int32),
        ("norm_eps", ctypes.c_float), ("emb_mult", ctypes.c_float), ("attn_scale", ctypes.c_float),
        ("resid_mult", ctypes.c_float), ("logits_scaling", ctypes.c_float),
    ]


class Weights(ctypes.Structure):
    _fields_ = [
        ("wqkv_q", ctypes.c_void_p), ("wqkv_sz", ctypes.c_void_p),
        ("wo_q", ctypes.c_void_p), ("wo_sz", ctypes.c_void_p),
        ("wgu_q", ctypes.c_void_p), ("wgu_sz", ctypes.c_void_p),
        ("wd_q", ctypes.c_void_p), ("wd_sz", ctypes.c_void_p),
        ("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p),
        ("final_norm", ctypes.c_void_p), ("embed", ctypes.c_void_p), ("rope", ctypes.c_void_p),
        ("rope_len", ctypes.c_int32),
        ("wqkv_t", ctypes.c_void_p), ("wo_t", ctypes.c_void_p),
        ("wgu_t", ctypes.c_void_p), ("wd_t", ctypes.c_void_p),
    ]


_lib = None


def load(path=LIB_PATH):
    """Load the shared library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: run `python -m flint_amd.build` (HIP library required)")
    lib = ctypes.CDLL(path)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
    sig = {
        "fl_version": ([], i32),
        "fl_device_info": ([vp, vp], i32),
        "fl_quantize_int4": ([vp, vp, vp, i32, i32, vp], i32),
        "fl_dequant_int4": ([vp, vp, vp, i32, i32, vp], i32),
        "fl_dequant_int4_mx": ([vp, vp, vp, i32, i32, vp], i32),
        "fl_gemv_int4": ([vp, vp, vp, vp, i32, i32, vp], i32),
        "fl_gemm_int4": ([vp, vp, vp, vp, i32, i32, i32, vp], i32),
        "fl_state_create": ([ctypes.POINTER(ModelDesc), i32, vp, vp, ctypes.POINTER(vp)], i32),
        "fl_state_destroy": ([vp], i32),
        "fl_state_reset": ([vp, vp], i32),
        "fl_state_check": ([vp, vp], i32),
        "fl_state_set_wait_limit": ([vp, ctypes.c_uint64], i32),
        "fl_state_force_timeout": ([vp, i32], i32),
        "fl_state_profile": ([vp, vp, i32, vp], i32),
        "fl_state_buffers": ([vp, vp, vp, vp, vp], i32),
        "fl_decode_step": ([ctypes.POINTER(Weights), vp, vp, i32, vp, vp, vp, vp], i32),
        "fl_decode_hidden": ([ctypes.POINTER(Weights), vp, vp, i32, vp, vp, vp, vp], i32),
        "fl_decode_sample": ([ctypes.POINTER(Weights), vp, vp, i32, f32, i32, ctypes.c_uint64, ctypes.c_uint64,
                              vp, vp, vp, vp], i32),
        "fl_verify": ([ctypes.POINTER(Weights), vp, vp, i32, vp, vp, i32, vp, vp, vp, vp], i32),
        "fl_kv_move": ([vp, vp, vp, i32, vp], i32),
        "fl_sample": ([vp, i32, i32, f32, i32, ctypes.c_uint64, ctypes.c_uint64, vp, vp, vp, vp], i32),
        "fl_sample_noalloc": ([vp, i32, i32, f32, i32, ctypes.c_uint64, ctypes.c_uint64, vp, vp, vp, vp], i32),
        "fl_probe_handoff": ([i32, i32, i32, vp, vp, vp], i32),
        "fl_tile_int4": ([vp, vp, i32, i32, vp], i32),
        "fl_dequant_int4_tiled": ([vp, vp, vp, i32, i32, vp], i32),
        "fl_gemv_int4_tiled": ([vp, vp, vp, vp, i32, i32, vp], i32),
        "fl_probe_dequant": ([i32, i32, vp, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def check(fn, code):
    if code != FL_OK:
        raise FlError(fn, code)
    return code


def call(name, *args):
    """Call a C-ABI entry point and raise FlError on a non-zero status."""
    lib = load()
    return check(name, getattr(lib, name)(*args))


def ptr(t):
    """Raw device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def device_view(ptr_value, n, dtype):
    """torch tensor viewing n elements of device memory owned by the library (diagnostics)."""
    import torch
    typestr = {torch.bfloat16: "<u2", torch.int32: "<i4", torch.int64: "<i8", torch.float32: "<f4"}[dtype]

    class _Arr:
        __cuda_array_interface__ = {"shape": (n,), "typestr": typestr,
                                    "data": (int(ptr_value), False), "version": 3}
    t = torch.as_tensor(_Arr(), device="cuda")
    return t.view(torch.bfloat16) if dtype == torch.bfloat16 else t
