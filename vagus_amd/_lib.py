"""ctypes binding of libvagus_gdr.so (the C ABI of include/vagus_gdr.h).

The library is loaded lazily on first use and there is no fallback: a missing
library raises RuntimeError with the build command, so a GPU run can never
silently execute something other than the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libvagus_gdr.so')

VGDR_OK, VGDR_ERR_INVALID, VGDR_ERR_UNSUPPORTED, VGDR_ERR_HIP = 0, 1, 2, 3
VGDR_F32, VGDR_BF16, VGDR_F16 = 0, 1, 2
VGDR_GATE_NONE, VGDR_GATE_SCALAR, VGDR_GATE_VECTOR = 0, 1, 2



class Fusion(ctypes.Structure):
    """struct vgdr_fusion: the producer fusions of a scan call."""
    _fields_ = [('qk_l2norm', ctypes.c_int), ('beta_sigmoid', ctypes.c_int), ('gate_activation', ctypes.c_int),
                ('gate_dtype', ctypes.c_int), ('A_log', ctypes.c_void_p), ('dt_bias', ctypes.c_void_p),
                ('lower_bound_set', ctypes.c_int), ('lower_bound', ctypes.c_float)]


class Epilogue(ctypes.Structure):
    """struct vgdr_epilogue: the layer's RMSNorm x SiLU(gate) output epilogue."""
    _fields_ = [('gate', ctypes.c_void_p), ('gamma', ctypes.c_void_p), ('gamma_dtype', ctypes.c_int),
                ('eps', ctypes.c_float)]


class ShortConv(ctypes.Structure):
    """struct vgdr_short_conv: the q, k, v short conv + SiLU and its decode caches."""
    _fields_ = [('weight_q', ctypes.c_void_p), ('weight_k', ctypes.c_void_p), ('weight_v', ctypes.c_void_p),
                ('cache_q', ctypes.c_void_p), ('cache_k', ctypes.c_void_p), ('cache_v', ctypes.c_void_p),
                ('kernel_size', ctypes.c_int), ('weight_dtype', ctypes.c_int)]


class GateProj(ctypes.Structure):
    """struct vgdr_gate_proj: the decode kernel's own scalar-gate and beta projections."""
    _fields_ = [('x', ctypes.c_void_p), ('w', ctypes.c_void_p), ('neg_exp_a', ctypes.c_void_p),
                ('dt_bias', ctypes.c_void_p), ('dim', ctypes.c_int64)]


# every symbol the header declares, with its ctypes signature
_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_FZ = ctypes.POINTER(Fusion)
_EP = ctypes.POINTER(Epilogue)
_SC = ctypes.POINTER(ShortConv)
_GP = ctypes.POINTER(GateProj)
SIGNATURES = {
    'vgdr_version': (_I, []),
    'vgdr_last_error': (ctypes.c_char_p, []),
    'vgdr_chunk_workspace_size': (_L, [_I, _I, _L, _L, _L, _L, _L, _I, _I]),
    'vgdr_chunk_fwd': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                            _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_prep': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                             _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_state': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                              _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_fwd_fused': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                  _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P]),
    'vgdr_chunk_prep_fused': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                   _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P]),
    'vgdr_chunk_fwd_noalloc': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P]),
    'vgdr_chunk_fwd_w': (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                              _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P]),
    'vgdr_chunk_bwd_workspace_size': (_L, [_I, _I, _L, _L, _L, _L, _L, _L, _I, _I]),
    'vgdr_chunk_bwd': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                            _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_bwd_saved': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                  _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_fwd_saving': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                   _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_fwd_saving_fused': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                         _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P]),
    'vgdr_chunk_bwd_fused': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                  _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P, _P, _P]),
    'vgdr_chunk_bwd_saved_fused': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                        _L, _L, _L, _L, _L, _L, _L, _F, _I, _FZ, _P, _P, _P]),
    'vgdr_chunk_bwd_w': (_I, [_I] + [_P] * 16 + [_L, _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_chunk_bwd_nodelta': (_I, [_I, _I] + [_P] * 14 + [_L, _L, _L, _L, _L, _L, _L, _F, _I, _P]),
    'vgdr_scan_bwd_workspace_size': (_L, [_L, _L, _L, _L, _L, _L]),
    'vgdr_scan_bwd': (_I, [_I, _I, _I] + [_P] * 18 + [_L, _L, _L, _L, _L, _L, _L, _F, _P]),
    'vgdr_recurrent_fwd': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                _L, _L, _L, _L, _L, _L, _F, _P]),
    'vgdr_recurrent_fwd_fused': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _L, _L, _L, _L, _L, _L, _F, _FZ, _P]),
    'vgdr_recurrent_fwd_epilogue': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                         _L, _L, _L, _L, _L, _L, _F, _FZ, _EP, _P]),
    'vgdr_norm_gate': (_I, [_I, _P, _EP, _P, _L, _L, _P]),
    'vgdr_rms_norm': (_I, [_I, _P, _P, _P, _P, _P, _L, _L, _F, _P]),
    'vgdr_scalar_gates': (_I, [_I, _P, _P, _P, _P, _P, _P, _L, _L, _L, _P]),
    'vgdr_swiglu': (_I, [_I, _P, _P, _L, _L, _P]),
    'vgdr_recurrent_fwd_w': (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                  _L, _L, _L, _L, _L, _L, _F, _FZ, _P]),
    'vgdr_decode_step': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                              _L, _L, _L, _L, _L, _L, _F, _FZ, _SC, _EP, _P]),
    'vgdr_decode_step_strided': (_I, [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _L, _L, _L, _L, _L, _L, _F, _FZ, _SC, _EP, _GP, _P]),
    'vgdr_causal_conv1d': (_I, [_I, _P, _P, _I, _P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _P]),
    'vgdr_varlen_workspace_size': (_L, [_L]),
    'vgdr_varlen_prepare': (_I, [_P, _L, _L, _I, _P, _P]),
}

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """The loaded library (cached).  Raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    with _lock:
        if _lib is not None and path == LIB_PATH:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(f'vagus_amd: {path} is not built; run `python -m vagus_amd.build` '
                               '(the HIP kernels are the only implementation)')
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path == LIB_PATH:
            _lib = lib
        return lib


def check(rc: int) -> None:
    """Map a status code to the reference's exception types
    (linear_attention.py:452-461: RuntimeError / NotImplementedError / AssertionError)."""
    if rc == VGDR_OK:
        return
    msg = load().vgdr_last_error().decode(errors='replace')
    if rc == VGDR_ERR_INVALID:
        raise AssertionError(msg)
    if rc == VGDR_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
