"""ctypes binding of ``libhla_s6.so`` (declared in ``include/hla_s6.h``).

torch is imported first so that the HIP runtime already loaded by torch (SONAME ``libamdhip64.so.7``) is the
one the library binds to: one runtime, one set of streams. A missing library is a hard error; there is no
fallback path.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get('HLA_S6_LIBRARY') or os.path.join(HERE, 'libhla_s6.so')   # override: another build
ABI_VERSION = 11

OK, EINVAL, EUNSUPPORTED, EWORKSPACE, ELAUNCH, EDEVICE = range(6)

P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float

# name -> argument types, in the order of include/hla_s6.h
SIGNATURES = {
    'hla_s6_abi_version': [],
    'hla_s6_last_error': [],
    'hla_s6_device_cus': [ctypes.c_int, ctypes.POINTER(ctypes.c_int)],
    'hla_s6_step_metadata': [P, I32, P, I32, I32, P, P, P, P, P, P, P],
    'hla_s6_gather_block_table': [P, I64, I32, I32, P, I32, P, I64, P],
    'hla_s6_latent_rope': [P, I32, I32, I32, I64, I64, P, P, I32, I64, P],
    'hla_s6_absorb': [P, I32, I32, I32, I64, I64, P, I64, I64, I32, P, I64, I64, P, P, I32, I64, P],
    'hla_s6_history_attention': [P, I32, I32, I32, I64, I64, P, P, I64, I64, I32, I64, P, I64, I32, P, P, F32, I32, P,
                                 I64, P, I64, I64, P, P],
    'hla_s6_history_attention_grouped': [P, I32, I32, I32, I64, I64, P, P, I64, I64, I32, I64, P, I64, I32, P, P, F32,
                                         I32, P, I64, P, I64, I64, P, I32, I32, P],
    'hla_s6_history_partials': [P, I32, I32, I32, I64, I64, P, P, I64, I64, I32, I64, P, I64, I32, P, P, F32, I32, P,
                                I64, P, I64, P],
    'hla_s6_history_reduce': [P, I64, I32, I32, I32, I32, P, I64, I64, P, P],
    'hla_s6_history_partials_grouped': [P, I32, I32, I32, I64, I64, P, P, I64, I64, I32, I64, P, I64, I32, P, P, F32,
                                        I32, P, I64, I32, P],
    'hla_s6_split_epilogue': [P, I64, I32, I32, I32, I32, P, I64, I64, P, P, P, P, I64, I64, P],
    'hla_s6_window_attention': [P, I32, I32, I32, I64, I64, P, P, I64, I64, I64, I32, I64, P, I64, I32, P, I32, P, P,
                                I32, P, I32, F32, P, I64, I64, P, P],
    'hla_s6_chunk_attention': [P, P, P, I32, I32, I32, I64, I64, I64, I64, I64, I64, P, I32, F32, P, I64, I64, P, P],
    'hla_s6_chunk_window_attention': [P, P, P, I32, I32, I32, I64, I64, I64, I64, I64, I64, P, P, I32, P, P, I64, I64,
                                      I64, I32, I64, P, I64, I32, I32, F32, P, I64, I64, P, P],
    'hla_s6_merge_states': [P, I64, I64, P, P, I64, I64, P, P, I32, I32, I32, I32, P, I64, I64, P, P],
    'hla_s6_attend_decode': [P, I64, I64, I32, P, P, I64, I64, I32, I64, P, I64, I32, P, P, P, I64, I64, P, P, I64, I64,
                             I64, I32, I64, P, I64, I32, P, P, I32, I32, P, I64, I64, P, I32, I32, F32, I32, I32, P,
                             I64, P, I64, P, P, P, P, P, I64, I64, P],
    'hla_s6_attend_decode_static': [P, I64, I64, I32, P, P, I64, I64, I32, I64, P, I64, I32, P, P, P, I64, I64, P, P,
                                    I64, I64, I64, I32, I64, P, I64, I32, P, P, I32, I32, P, I64, I64, P, I32, I32,
                                    F32, I32, I32, P, I64, I64, P],
    'hla_s6_split_plan_ints': [I32, I32],
    'hla_s6_split_plan': [P, I32, I64, I32, P, I32, P, I64, P],
    'hla_s6_split_plans': [P, I32, I64, I32, P, P, I32, P, P, P],
    'hla_s6_slot_mapping': [P, I64, I32, P, P, P, I32, I32, P, P],
    'hla_s6_store_rows': [P, I64, P, I64, I32, I32, P, P, I64, I64, I32, I64, P],
    'hla_s6_write_rows': [P, I32, I32, I64, P, I32, I64, P, I64, P, I64, P, P, P, I32, I64, P, I64, I64, I32, I64, P],
    'hla_s6_gather_packed_rows': [P, I32, I64, I64, I32, I64, P, I32, I64, I64, I32, I64, P, I32, I32, P, I64, I64, I32,
                                  P],
    'hla_s6_khop_bounds': [P, I64, I64, I32, I32, I32, P, P],
    'hla_s6_khop_forward': [P, I64, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I32, I32, I32, I32, I32, F32, P,
                            I64, I64, I64, P, P],
    'hla_s6_masked_history': [P, I64, I64, P, P, I64, I64, P, I64, P, I32, I32, I32, I32, F32, I32, P, I64, P, I64,
                              I64, P, P],
    'hla_s6_hf_chunk_forward': [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64, P, I64, I32, I32, I32, I32, F32,
                                P, I64, I64, I64, P, I64, I64, P],
    'hla_s6_hf_chunk_backward': [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64, P, I64, I32, I32, I32, I32,
                                 F32, P, I64, I64, I64, P, I64, I64, P, I64, I64, I64, P, P, P, P, P, I64, I64, I64, P],
    'hla_s6_khop_backward_workspace': [I32, I32, I32, I32, I32],
    'hla_s6_khop_backward': [P, I64, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I32, I32, I32, I32, I32, F32,
                             P, I64, I64, I64, P, P, I64, I64, I64, P, P, P, I64, I64, I64, P, I64, I64, P, I64, I64,
                             I32, P, I64, I32, P],
    'hla_s6_khop_forward_f32': [P, I64, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I32, I32, I32, I32, I32,
                                F32, P, I64, I64, I64, P, P],
    'hla_s6_khop_backward_f32_workspace': [I32, I32, I32, I32, I32],
    'hla_s6_khop_backward_f32': [P, I64, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, P, I32, I32, I32, I32, I32,
                                 F32, P, I64, I64, I64, P, P, I64, I64, I64, P, P, P, I64, I64, I64, P, I64, I64, P,
                                 I64, I64, I32, P, I64, P],
    'hla_s6_mixed_merge_forward': [I32, I32, I32, I32, I32, P, I64, I64, I64, P, I32, P, P, P, P, I64, I64, P, I64,
                                   I64, I64, P],
    'hla_s6_mixed_merge_backward': [I32, I32, I32, I32, I32, P, I64, I64, I64, P, I32, P, P, P, P, I64, I64, P, I64,
                                    I64, I64, P, I64, I64, I64, P, P, P, P, P],
    'hla_s6_rope_rows_forward': [I32, P, P, P, P, I32, I32, I32, I32, P, P, I64, I64, I32, P],
    'hla_s6_rope_rows_backward': [I32, P, P, P, P, I32, I32, I32, I32, P, P, I64, I64, I32, P],
}

RESTYPES = {'hla_s6_last_error': ctypes.c_char_p, 'hla_s6_split_plan_ints': ctypes.c_int64,
            'hla_s6_khop_backward_workspace': ctypes.c_int64, 'hla_s6_khop_backward_f32_workspace': ctypes.c_int64}

_LIB = None


def load() -> ctypes.CDLL:
    """The loaded library (loaded once); raises RuntimeError when it is missing or of another ABI."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f'{LIB_PATH} is missing: build it first (python __graft_entry__.py build, or '
                               f'python hybrid-latent-attention_amd/build.py); the S6 path has no fallback')
        lib = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        version = lib.hla_s6_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f'libhla_s6.so ABI {version}, expected {ABI_VERSION}: rebuild the library')
        _LIB = lib
    return _LIB


def check(rc: int) -> None:
    """Map a status code to the exception type the reference op raises for the same condition."""
    if rc == OK:
        return
    msg = load().hla_s6_last_error().decode(errors='replace')
    if rc in (EINVAL, EUNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def ptr(t) -> int | None:
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream(device=None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


_CUS: dict = {}


def device_cus(device: int = 0) -> int:
    """Compute units of HIP device ``device`` (queried once per device)."""
    if device not in _CUS:
        out = ctypes.c_int(0)
        check(load().hla_s6_device_cus(device, ctypes.byref(out)))
        _CUS[device] = out.value
    return _CUS[device]
