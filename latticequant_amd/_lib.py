"""Loader for liblatticequant_amd.so (the gfx950 kernels behind a C ABI).

torch is imported first on purpose: torch ships its own libamdhip64.so.7 and
the kernel library links against that soname, so loading it after torch binds
it to torch's HIP runtime (one runtime per process, shared streams and
pointers).  The library is required: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblatticequant_amd.so")

LQ_L = 1024
LQ_BLK = 512
LQ_ESC_MAX_SHIFT = 7
LQ_SYM_STRIDE = 4352
LQ_MAXSYM = 1028
LQ_STREAMS = 16
LQ_F16, LQ_BF16, LQ_F32 = 0, 1, 2
LQ_ST_SYM_OVERFLOW, LQ_ST_ALPHABET, LQ_ST_TIE_UNPINNED = 1, 2, 4
LQ_V_VALID, LQ_V_HALF, LQ_V_INRANGE = 1, 2, 4
TABLE_BYTES = 16 + 4 * LQ_MAXSYM   # sizeof(lq_table)

_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int

_SIGS = {
    "lq_version": ([], _INT),
    "lq_hip_runtime_version": ([], _INT),
    "lq_status_string": ([_INT], ctypes.c_char_p),
    "lq_e8_encode_f32": ([_P, _I64, _INT, _P, _P], _INT),
    "lq_e8_to_symbols": ([_P, _I64, _P, _P, _P], _INT),
    "lq_symbols_to_e8": ([_P, _P, _I64, _P, _P], _INT),
    "lq_head_scales": ([_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_quantize_deq_workspace": ([_I64, _I64, _I64], _I64),
    "lq_quantize_deq": ([_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_scale_fastdiv": ([_P, _I64, _INT, _P, _P], _INT),
    "lq_chunk_quantize": ([_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _INT, _P, _P], _INT),
    "lq_chunk_tables": ([_P, _I64, _P, _P, _P], _INT),
    "lq_chunk_quantize_wide": ([_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _INT, _P, _P], _INT),
    "lq_chunk_hist_wide": ([_P, _P, _I64, _I64, _P, _P, _P], _INT),
    "lq_chunk_escape_plan": ([_P, _I64, _P, _P, _P, _P], _INT),
    "lq_chunk_escape_split": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _P], _INT),
    "lq_chunk_decode_escaped": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P,
                                 _INT, _P, _P], _INT),
    "lq_chunk_tables_wide": ([_P, _P, _I64, _P, _P, _P], _INT),
    "lq_chunk_encode_wide": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_chunk_encode_workspace": ([_I64, _I64], _I64),
    "lq_chunk_encode": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_chunk_pack": ([_I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_chunk_decode": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _INT, _P, _P], _INT),
    "lq_build_tables": ([_P, _P, _P, _I32, _P, _P, _P, _P, _P], _INT),
    "lq_rans_encode_streams": ([_P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P], _INT),
    "lq_rans_decode_streams": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _I32, _P, _P], _INT),
    "lq_unpack_compact": ([_P, _INT, _I64, _P, _I64, _P, _P, _P], _INT),
    "lq_pack_compact": ([_P, _INT, _I64, _P, _P, _P], _INT),
    "lq_merge_workspace": ([_I64], _I64),
    "lq_compact_encode_workspace": ([_I64], _I64),
    "lq_compact_encode": ([_P, _INT, _I64, _I64, _P, _P, _P, _INT, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_compact_encode_scaled_workspace": ([_I64, _I64], _I64),
    "lq_compact_encode_scaled": ([_P, _INT, _I64, _I64, _INT, _INT, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
                                 _INT),
    "lq_compact_merge": ([_P, _I64, _INT, _P, _I64, _P, _P, _I64, _I64, _P, _P, _P], _INT),
    "lq_fused_merge": ([_P, _I64, _INT, _P, _I64, _P, _P, _I64, _I64, _P, _P, _P], _INT),
    "lq_e8_validate": ([_P, _I64, ctypes.c_float, _INT, _P, _P], _INT),
    "lq_unpack_e8": ([_P, _INT, _I64, _P, _P], _INT),
    "lq_symbol_index": ([_P, _I64, _P, _I32, _INT, _P, _P], _INT),
    "lq_pack_coset_bits": ([_P, _I64, _P, _P], _INT),
    "lq_unpack_coset_bits": ([_P, _I64, _P, _P], _INT),
    "lq_e8_quantize_heads": ([_P, _INT, _I64, _I64, _P, _P, _P, _P], _INT),
    "lq_chunk_luts": ([_P, _I64, _P, _P], _INT),
    "lq_attn_workspace": ([_I64, _I64, _I64, _INT], _I64),
    "lq_decode_attention": ([_P, _P, _P, _INT, _P, _P, _I64, _P, _P, _P], _INT),
    "lq_rht": ([_P, _INT, _I64, _INT, _P, _I64, _INT, _INT, _P, _INT, _P], _INT),
    "lq_head_scales_rht": ([_P, _INT, _I64, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_chunk_quantize_rht": ([_P, _INT, _I64, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P, _P, _P, _P], _INT),
    "lq_chunk_decode_rht": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _P, _INT, _P, _P], _INT),
    "lq_resident_workspace": ([_I64, _I64], _I64),
    "lq_resident_quantize": ([_P, _INT, _I64, _I64, _P, _P, _P, _I64, _I64, _P, _P], _INT),
    "lq_resident_dequant": ([_P, _I64, _I64, _I64, _I64, _P, _INT, _P], _INT),
    "lq_resident_attn_workspace": ([_I64, _INT, _I64, _I64], _I64),
    "lq_resident_attention": ([_P, _P, _I64, _P, _INT, _P, _P, _I64, _P, _P, _P], _INT),
    "lq_resident_attention_noalloc": ([_P, _P, _I64, _P, _INT, _P, _P, _I64, _P, _P], _INT),
}


class LQError(RuntimeError):
    pass


class ChunkBatch(ctypes.Structure):
    """lq_chunk_batch: device pointers + geometry of one chunk batch."""
    _fields_ = [("words", _P), ("chunk_base", _P), ("stream_woff", _P), ("blk_off", _P), ("stream_nbits", _P), ("blk_state", _P),
                ("coset_bits", _P), ("blk_n1", _P), ("tables", _P), ("scale16", _P),
                ("n_chunks", _I64), ("n_heads", _I64), ("bph", _I64)]


class Resident(ctypes.Structure):
    """lq_resident: device pointers + geometry of a resident (fixed-width) KV prefix."""
    _fields_ = [("a", _P), ("b", _P), ("mask", _P), ("meta", _P), ("exc", _P), ("scale", _P), ("n_exc", _P),
                ("status", _P), ("n_heads", _I64), ("cap_blocks", _I64), ("exc_cap", _I64)]


LQ_RES_ST_EXC_OVERFLOW = 1


def exported_symbols():
    """Names the C ABI exports (declared in include/latticequant_amd.h)."""
    return sorted(_SIGS)


def load(path: str = LIB_PATH):
    """Load the kernel library (once).  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LQError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                      "(hipcc --offload-arch=gfx950); latticequant_amd has no CPU fallback")
    lib = ctypes.CDLL(path)
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def check_runtime():
    """The library must run on torch's HIP runtime (same process-wide instance)."""
    lib = load()
    if not torch.cuda.is_available():
        raise LQError("latticequant_amd needs a ROCm GPU (gfx950); none is visible")
    torch.cuda.init()
    v = lib.lq_hip_runtime_version()
    want = torch.version.hip
    if v < 0 or want is None:
        raise LQError(f"HIP runtime check failed (lib reports {v}, torch {want})")
    major, minor = v // 10000000, (v // 100000) % 100
    tmaj, tmin = (int(t) for t in want.split(".")[:2])
    if (major, minor) != (tmaj, tmin):
        raise LQError(f"kernel library bound to HIP {major}.{minor} but torch uses {want}: two runtimes in one process")
    return v


_checked = False


def lib():
    """Library handle for GPU work (runtime verified on first use)."""
    global _checked
    l = load()
    if not _checked:
        check_runtime()
        _checked = True
    return l


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def debug_checks() -> bool:
    """LQ_DEBUG_CHECKS=1: wrappers also validate device-side index ranges on
    the host (each such check syncs with the device); by default they rely on
    the kernels' own clamping."""
    return os.environ.get("LQ_DEBUG_CHECKS", "") not in ("", "0")


def check(rc: int, what: str):
    if rc != 0:
        msg = load().lq_status_string(rc).decode()
        raise LQError(f"{what} failed: {msg} ({rc})")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float16:
        return LQ_F16
    if dt == torch.bfloat16:
        return LQ_BF16
    if dt == torch.float32:
        return LQ_F32
    raise LQError(f"unsupported dtype {dt}; expected float16, bfloat16 or float32")
