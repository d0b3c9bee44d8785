"""ctypes binding of libdetllm_amd.so (the C ABI in include/detllm.h).

The library is built in-tree by detllm_amd.build.  Loading never falls back
to anything else: if the shared object is missing the import of this module
raises, so no product path can silently run on the CPU.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from .build import LIB_NAME, OUT_DIR

LIB_PATH = OUT_DIR / LIB_NAME


class DetllmError(RuntimeError):
    """A non-zero dtl_status returned by the library."""

    def __init__(self, status: int, where: str):
        self.status = status
        self.where = where
        super().__init__(f"{where}: {status_name(status)} (status {status})")


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m detllm_amd.build` "
            "(the HIP implementation is required; there is no CPU fallback)"
        )
    return C.CDLL(str(LIB_PATH))


# With at least five hardware queues per process the pipelined encode keeps
# four chunks in flight on four streams, else three (HIP's default is four
# queues).  Eight queues unless the caller chose otherwise; HIP reads the
# setting when it initialises, i.e. at the library's first HIP call.
os.environ.setdefault("GPU_MAX_HW_QUEUES", "8")
lib = _load()

u8p = C.POINTER(C.c_uint8)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
u16p = C.POINTER(C.c_uint16)
vpp = C.POINTER(C.c_void_p)
sz = C.c_size_t


class ModelConfig(C.Structure):
    _fields_ = [
        ("block_count", C.c_uint64),
        ("embedding_length", C.c_uint64),
        ("feed_forward_length", C.c_uint64),
        ("head_count", C.c_uint64),
        ("head_count_kv", C.c_uint64),
        ("head_dim", C.c_uint64),
        ("rope_dimension_count", C.c_uint64),
        ("context_length", C.c_uint64),
        ("vocab", C.c_uint64),
        ("rms_epsilon", C.c_float),
        ("attention_scale", C.c_float),
        ("rope_freq_base", C.c_float),
        ("rope_split_half", C.c_int32),
        ("embedding_type", C.c_int32),
        ("output_type", C.c_int32),
        ("has_qkv_bias", C.c_int32),
        ("device_bytes", C.c_uint64),
    ]


class RangeDecoderState(C.Structure):
    """dtl_range_decoder_state: low, range, code and the input bytes consumed."""

    _fields_ = [("low", C.c_uint64), ("range", C.c_uint64), ("code", C.c_uint64), ("pos", C.c_uint64)]


class KernelStat(C.Structure):
    _fields_ = [
        ("name", C.c_char * 32),
        ("launches", C.c_uint64),
        ("total_ms", C.c_double),
        ("bytes", C.c_double),
        ("macs", C.c_double),
    ]


_SIGS = {
    "dtl_status_string": (C.c_char_p, [C.c_int]),
    "dtl_model_load": (C.c_int, [C.c_char_p, sz, vpp]),
    "dtl_model_free": (None, [C.c_void_p]),
    "dtl_model_get_config": (C.c_int, [C.c_void_p, C.POINTER(ModelConfig)]),
    "dtl_session_new": (C.c_int, [C.c_void_p, sz, sz, vpp]),
    "dtl_session_free": (None, [C.c_void_p]),
    "dtl_session_reset": (C.c_int, [C.c_void_p]),
    "dtl_forward_one": (C.c_int, [C.c_void_p, C.c_uint32, sz, f32p]),
    "dtl_forward_chunk": (C.c_int, [C.c_void_p, u32p, sz, sz, f32p]),
    "dtl_session_logits": (C.c_int, [C.c_void_p, sz, sz, f32p]),
    "dtl_logits_hash": (C.c_int, [C.c_void_p, u32p, sz, sz, u8p]),
    "dtl_session_set_profiling": (C.c_int, [C.c_void_p, C.c_int]),
    "dtl_session_profile": (C.c_int, [C.c_void_p, C.POINTER(KernelStat), sz, C.POINTER(sz)]),
    "dtl_session_profile_only": (C.c_int, [C.c_void_p, C.c_char_p]),
    "dtl_session_get_info": (C.c_int, [C.c_void_p, C.POINTER(sz), C.POINTER(sz), C.POINTER(sz)]),
    "dtl_symbol_ranges": (C.c_int, [C.c_void_p, sz, sz, u32p, sz, u64p, u32p, u64p]),
    "dtl_symbol_ranges_rows": (C.c_int, [C.c_void_p, sz, u32p, u32p, sz, u64p, u32p, u64p]),
    "dtl_forward_ranges": (C.c_int, [C.c_void_p, u32p, sz, sz, sz, u32p, u32p, sz, u64p, u32p, u64p]),
    "dtl_cdf": (C.c_int, [C.c_void_p, sz, sz, u32p, u64p, u64p]),
    "dtl_decoder_total": (C.c_int, [C.c_void_p, sz, sz, u64p]),
    "dtl_decoder_lookup": (C.c_int, [C.c_void_p, sz, sz, C.c_uint64, u32p, u64p, u32p, u64p]),
    "dtl_decoder_decode": (C.c_int, [C.c_void_p, sz, sz, C.c_void_p, u32p]),
    "dtl_forward_decode": (C.c_int, [C.c_void_p, C.c_uint32, sz, sz, C.c_void_p, u32p]),
    "dtl_logits_to_cdf": (C.c_int, [f32p, sz, sz, u32p, u64p, u64p]),
    "dtl_logits_to_symbol_range": (C.c_int, [f32p, sz, sz, sz, u64p, u32p, u64p]),
    "dtl_uniform_cdf": (C.c_int, [sz, u32p, u64p, u64p]),
    "dtl_uniform_symbol_range": (C.c_int, [sz, sz, u64p, u32p, u64p]),
    # device pointers throughout (logits, symbols, cum, freq, total, status word, stream)
    "dtl_symbol_ranges_static": (C.c_int, [C.c_void_p, sz, sz, C.c_void_p, sz, C.c_void_p, C.c_void_p,
                                           C.c_void_p, C.c_void_p, C.c_void_p]),
    "dtl_status_from_bits": (C.c_int, [C.c_int]),
    "dtl_range_encoder_new": (C.c_int, [vpp]),
    "dtl_range_encode": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64]),
    "dtl_range_encoder_finish": (C.c_int, [C.c_void_p, u8p, sz, C.POINTER(sz)]),
    "dtl_range_encoder_free": (None, [C.c_void_p]),
    "dtl_range_encoder_snapshot": (C.c_int, [C.c_void_p, u64p, u64p, u8p, sz, C.POINTER(sz)]),
    "dtl_range_encoder_from_snapshot": (C.c_int, [C.c_uint64, C.c_uint64, u8p, sz, vpp]),
    "dtl_range_decoder_new": (C.c_int, [u8p, sz, vpp]),
    "dtl_range_decode_freq": (C.c_int, [C.c_void_p, C.c_uint64, u64p]),
    "dtl_range_decode_advance": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64]),
    "dtl_range_decoder_free": (None, [C.c_void_p]),
    "dtl_range_decoder_snapshot": (C.c_int, [C.c_void_p, C.POINTER(RangeDecoderState)]),
    "dtl_range_decoder_from_snapshot": (C.c_int, [u8p, sz, C.POINTER(RangeDecoderState), vpp]),
    "dtl_tokenizer_from_gguf": (C.c_int, [C.c_char_p, sz, vpp]),
    "dtl_tokenizer_free": (None, [C.c_void_p]),
    "dtl_tokenizer_vocab_len": (sz, [C.c_void_p]),
    "dtl_tokenizer_codec_symbols": (C.c_int, [C.c_void_p, u8p, sz, sz, u32p, sz, C.POINTER(sz)]),
    "dtl_tokenizer_decode_symbol": (C.c_int, [C.c_void_p, C.c_uint32, sz, u8p, sz, C.POINTER(sz)]),
    "dtl_codec_next_window_start": (sz, [sz, sz, sz, sz]),
    "dtl_codec_encode": (C.c_int, [C.c_void_p, u32p, sz, sz, C.c_int, u8p, sz, C.POINTER(sz)]),
    "dtl_codec_decode": (
        C.c_int,
        [C.c_void_p, u8p, sz, sz, C.c_int, u8p, sz, sz, u32p, C.POINTER(sz)],
    ),
    "dtl_dtlz_header_encode": (C.c_int, [C.c_uint16, u8p, C.c_uint32, C.c_uint32, C.c_uint64, u8p]),
    "dtl_dtlz_header_decode": (
        C.c_int,
        [u8p, sz, u16p, u8p, u32p, u32p, u64p],
    ),
    "dtl_compress": (C.c_int, [C.c_void_p, C.c_void_p, u8p, u8p, sz, sz, sz, C.POINTER(u8p), C.POINTER(sz)]),
    "dtl_decompress": (C.c_int, [C.c_void_p, C.c_void_p, u8p, u8p, sz, sz, C.POINTER(u8p), C.POINTER(sz)]),
    "dtl_decompress_part": (
        C.c_int,
        [C.c_void_p, C.c_void_p, u8p, u8p, sz, sz, u32p, sz, C.POINTER(RangeDecoderState), sz, u32p, sz,
         C.POINTER(sz), C.POINTER(RangeDecoderState), C.POINTER(C.c_int), C.POINTER(u8p), C.POINTER(sz)],
    ),
    "dtl_bytes_free": (None, [u8p]),
    "dtl_kernel_exp_f32": (C.c_int, [f32p, f32p, sz]),
    "dtl_kernel_silu_f32": (C.c_int, [f32p, f32p, sz]),
    "dtl_kernel_exp_clamped_f32": (C.c_int, [f32p, f32p, sz]),
    "dtl_valu_probe": (C.c_int, [C.POINTER(C.c_double)]),
    "dtl_mfp_probe": (C.c_int, [C.POINTER(C.c_double)]),
    "dtl_kernel_f16_to_f32": (C.c_int, [u16p, f32p, sz]),
    "dtl_kernel_div_sqrt": (C.c_int, [f32p, f32p, f32p, f32p, sz]),
    "dtl_kernel_quantize": (C.c_int, [f32p, sz, sz, f32p, i8p, f32p, i8p]),
    "dtl_kernel_rmsnorm": (C.c_int, [f32p, f32p, C.c_float, sz, sz, f32p]),
    "dtl_kernel_gemv": (C.c_int, [C.c_int, u8p, sz, sz, f32p, sz, f32p]),
    "dtl_kernel_q4k_chunk": (C.c_int, [C.c_int, C.c_int, u8p, sz, u8p, sz, sz, f32p, sz, f32p, f32p]),
    "dtl_kernel_rope_table": (C.c_int, [C.c_float, sz, sz, f32p, f32p]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = tuple(_SIGS)


def status_name(status: int) -> str:
    return lib.dtl_status_string(status).decode()


def check(status: int, where: str) -> None:
    if status != 0:
        raise DetllmError(status, where)


def ptr(arr, ctype):
    """Pointer to a contiguous numpy array's data."""
    return arr.ctypes.data_as(C.POINTER(ctype))
