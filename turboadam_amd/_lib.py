"""ctypes binding of libturboadam_amd.so (C ABI declared in include/turboadam_amd.h).

The library is loaded after torch, so its HIP runtime dependency
(soname libamdhip64.so.7) resolves to the runtime torch already mapped and
kernels run on torch's streams and allocations.  There is no fallback: if the
library is missing or a second HIP runtime would be mapped, loading raises.
"""

import ctypes
import os

import torch  # noqa: F401  (must be imported before the HIP library is mapped)

from .build import LIB_PATH

TAM_DTYPE_F32 = 0
TAM_DTYPE_BF16 = 1
TAM_DTYPE_F16 = 2

# torch dtype of a parameter / gradient -> TAM_DTYPE_*
DTYPES = {torch.float32: TAM_DTYPE_F32, torch.bfloat16: TAM_DTYPE_BF16, torch.float16: TAM_DTYPE_F16}

TAM_FLAG_COSTATE = 0x1
TAM_FLAG_COMPRESS_V = 0x2
TAM_FLAG_HAS_STATE = 0x4
TAM_FLAG_WD = 0x8
TAM_FLAG_EF = 0x10
TAM_FLAG_HAS_EF = 0x20
TAM_FLAG_DEVICE_STEP = 0x40

ABI_VERSION = 8
# workspace of tam_multi_tensor_step_static (include/turboadam_amd.h)
TAM_STATIC_SCRATCH_BYTES = 64 << 20


class TamTensor(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("v_idx", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("signs", ctypes.c_void_p),
        ("labels", ctypes.c_void_p),
        ("norms", ctypes.c_void_p),
        ("amp", ctypes.c_void_p),
        ("alpha", ctypes.c_void_p),
        ("n", ctypes.c_uint64),
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("v_bits", ctypes.c_uint32),
        ("tensor_id", ctypes.c_uint32),
        ("step", ctypes.c_uint32),
        ("k_lo", ctypes.c_uint32),
        ("k_hi", ctypes.c_uint32),
        ("inv_bc2_f32", ctypes.c_float),
        ("c_wd", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("one_minus_beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("bias_correction1", ctypes.c_float),
        ("bias_correction2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("neg_lr", ctypes.c_float),
        ("sqrt_block", ctypes.c_float),
        ("nb", ctypes.c_uint32),
        ("tile0", ctypes.c_uint32),
        ("ntiles", ctypes.c_uint32),
        ("chunk0", ctypes.c_uint32),
        ("ratio_off", ctypes.c_uint64),
        ("inv_bc2", ctypes.c_double),
        ("slice0", ctypes.c_uint32),
        ("c_lr", ctypes.c_float),
        ("ef_residual", ctypes.c_void_p),
        ("ef_off", ctypes.c_uint64),
        ("step_dev", ctypes.c_void_p),
        ("bc_step", ctypes.c_void_p),
        ("bc_table", ctypes.c_void_p),
        ("bc_len", ctypes.c_uint32),
        ("k_abs", ctypes.c_float),
        ("found_inf", ctypes.c_void_p),
        ("tail0", ctypes.c_uint32),
        ("tail_wgs", ctypes.c_uint32),
    ]


class TamStepInfo(ctypes.Structure):
    _fields_ = [
        ("n_tensors", ctypes.c_int32),
        ("total_tiles", ctypes.c_uint32),
        ("n_costate", ctypes.c_uint32),
        ("total_chunks", ctypes.c_uint32),
        ("total_slices", ctypes.c_uint32),
        ("dtype_mask", ctypes.c_uint32),
        ("ratio_blocks", ctypes.c_uint64),
        ("off_partials", ctypes.c_uint64),
        ("off_alpha", ctypes.c_uint64),
        ("off_ratios", ctypes.c_uint64),
        ("ws_bytes", ctypes.c_uint64),
        ("off_chunks", ctypes.c_uint64),
        ("off_sel", ctypes.c_uint64),
        ("off_hist", ctypes.c_uint64),
        ("n_ef", ctypes.c_uint32),
        ("n_device_step", ctypes.c_uint32),
        ("off_ef_alpha", ctypes.c_uint64),
        ("tail_blocks", ctypes.c_uint32),
    ]


# Every symbol include/turboadam_amd.h declares, with its ctypes signature.
_VP = ctypes.c_void_p
SIGNATURES = {
    "tam_abi_version": (ctypes.c_int, []),
    "tam_struct_size": (ctypes.c_size_t, [ctypes.c_int]),
    "tam_last_error": (ctypes.c_char_p, []),
    "tam_prepare": (ctypes.c_int, [ctypes.POINTER(TamTensor), ctypes.c_int, ctypes.POINTER(TamStepInfo)]),
    "tam_multi_tensor_step": (
        ctypes.c_int,
        [_VP, ctypes.POINTER(TamTensor), ctypes.POINTER(TamStepInfo), ctypes.c_uint64, _VP, ctypes.c_size_t, _VP],
    ),
    "tam_multi_tensor_step_static": (
        ctypes.c_int,
        [_VP, ctypes.POINTER(TamTensor), ctypes.POINTER(TamStepInfo), ctypes.c_uint64, _VP],
    ),
    "tam_step_pass": (
        ctypes.c_int,
        [ctypes.c_int, _VP, ctypes.POINTER(TamStepInfo), ctypes.c_uint64, _VP, ctypes.c_size_t, _VP],
    ),
    "tam_v_dequantize": (ctypes.c_int, [_VP, _VP, ctypes.c_uint64, ctypes.c_uint32, _VP, _VP]),
    "tam_philox_uniforms": (
        ctypes.c_int,
        [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, _VP, _VP],
    ),
    "tam_math_eval": (ctypes.c_int, [ctypes.c_int, _VP, _VP, ctypes.c_uint64, _VP]),
    "tam_costate_decode": (
        ctypes.c_int,
        [_VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_float,
         ctypes.c_float, _VP, _VP],
    ),
    "tam_decompose_workspace": (ctypes.c_size_t, [ctypes.c_uint64]),
    "tam_decompose": (ctypes.c_int, [_VP, _VP, ctypes.c_uint64, _VP, _VP, _VP, ctypes.c_size_t, _VP]),
    "tam_block_ratios": (ctypes.c_int, [_VP, _VP, ctypes.c_uint64, _VP, _VP]),
    "tam_thresholds_workspace": (ctypes.c_size_t, [ctypes.c_uint64]),
    "tam_thresholds": (
        ctypes.c_int,
        [_VP, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, _VP, _VP, ctypes.c_size_t, _VP],
    ),
    "tam_classify": (ctypes.c_int, [_VP, ctypes.c_uint64, _VP, _VP, _VP]),
    "tam_costate_encode": (ctypes.c_int, [_VP, ctypes.c_uint64, _VP, _VP, _VP, _VP]),
    "tam_fused_v_update": (
        ctypes.c_int,
        [_VP, _VP, _VP, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, ctypes.c_float,
         ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, _VP, _VP, _VP, _VP],
    ),
    "tam_v_quantize": (
        ctypes.c_int,
        [_VP, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, _VP,
         _VP, _VP],
    ),
}

_lib = None


def _hip_runtimes_mapped():
    paths = set()
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                parts = line.split()
                if len(parts) >= 6 and "libamdhip64.so" in parts[-1]:
                    paths.add(os.path.realpath(parts[-1]))
    except OSError:
        pass
    return paths


def load(path: str = None) -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing or broken."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(
            f"turboadam_amd: HIP library not built ({path}); run turboadam_amd.build.build_library()"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.tam_abi_version() != ABI_VERSION:
        raise RuntimeError("turboadam_amd: ABI version mismatch")
    if lib.tam_struct_size(0) != ctypes.sizeof(TamTensor) or lib.tam_struct_size(1) != ctypes.sizeof(TamStepInfo):
        raise RuntimeError("turboadam_amd: struct layout mismatch between library and binding")
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"turboadam_amd: more than one HIP runtime mapped: {sorted(runtimes)}")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.tam_last_error().decode() if _lib is not None else ""
        raise RuntimeError(f"turboadam_amd: {what} failed (code {rc}): {msg}")


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
