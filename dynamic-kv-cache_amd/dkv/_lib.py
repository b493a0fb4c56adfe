"""ctypes binding of libdkv.so, the C ABI declared in include/dkv.h.

torch is imported first on purpose: torch ships its own HIP runtime, and the
library must bind to that same runtime so that torch's stream handles are valid
in it. There is no fallback path: if the library is missing, every entry point
raises.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

from . import _build

DKV_EINVAL = -1
DKV_MAX_CHUNK_SEGS = 16
DKV_ARG_TILES = 128  # tile descriptors a launch can carry in its argument block (include/dkv.h)
DKV_NOALLOC_SCRATCH_BYTES = 16 << 20
ABI_VERSION = 3


class Tile(ctypes.Structure):
    _fields_ = [('offset', ctypes.c_int64), ('token_start', ctypes.c_int32),
                ('rows', ctypes.c_uint16), ('bits', ctypes.c_uint8), ('reserved', ctypes.c_uint8)]


class PackJob(ctypes.Structure):
    _fields_ = [('k', ctypes.c_void_p), ('v', ctypes.c_void_p),
                ('k_head_stride', ctypes.c_int64), ('k_tok_stride', ctypes.c_int64),
                ('v_head_stride', ctypes.c_int64), ('v_tok_stride', ctypes.c_int64),
                ('seg_offset', ctypes.c_int64), ('seg_rows', ctypes.c_int32),
                ('seg_token_start', ctypes.c_int32), ('row0', ctypes.c_int32), ('n', ctypes.c_int32),
                ('layer', ctypes.c_int32), ('bits', ctypes.c_int32), ('tile_index0', ctypes.c_int32),
                ('write_tiles', ctypes.c_int32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [('q', ctypes.c_void_p), ('q_head_stride', ctypes.c_int64), ('q_tok_stride', ctypes.c_int64),
                ('k_new', ctypes.c_void_p), ('kn_head_stride', ctypes.c_int64), ('kn_tok_stride', ctypes.c_int64),
                ('v_new', ctypes.c_void_p), ('vn_head_stride', ctypes.c_int64), ('vn_tok_stride', ctypes.c_int64),
                ('arena', ctypes.c_void_p), ('tiles', ctypes.c_void_p),
                ('n_tiles', ctypes.c_int32), ('past', ctypes.c_int32),
                ('layer', ctypes.c_int32), ('layers', ctypes.c_int32), ('heads', ctypes.c_int32),
                ('q_heads', ctypes.c_int32), ('nq', ctypes.c_int32),
                ('n_segs', ctypes.c_int32), ('seg_bounds', ctypes.c_int32 * (DKV_MAX_CHUNK_SEGS + 1)),
                ('scale', ctypes.c_float),
                ('out', ctypes.c_void_p), ('out_tok_stride', ctypes.c_int64), ('out_head_stride', ctypes.c_int64),
                ('out_dtype', ctypes.c_int32), ('path', ctypes.c_int32), ('splits', ctypes.c_int32),
                ('precision', ctypes.c_int32),
                ('workspace', ctypes.c_void_p), ('workspace_bytes', ctypes.c_int64),
                ('step', ctypes.c_void_p), ('tiles_host', ctypes.c_void_p)]


class SegmentIO(ctypes.Structure):
    _fields_ = [('payload', ctypes.c_void_p * 2), ('offsets', ctypes.c_void_p * 2), ('scales', ctypes.c_void_p * 2),
                ('seg_offset', ctypes.c_int64), ('seg_rows', ctypes.c_int32), ('seg_token_start', ctypes.c_int32),
                ('row0', ctypes.c_int32), ('rows', ctypes.c_int32), ('bits', ctypes.c_int32),
                ('layer0', ctypes.c_int32), ('n_layers', ctypes.c_int32), ('tile_index0', ctypes.c_int32),
                ('write_tiles', ctypes.c_int32)]


assert ctypes.sizeof(Tile) == 16

_lib = None

# (name, restype, argtypes) of every symbol include/dkv.h declares.
SIGNATURES = [
    ('dkv_version', ctypes.c_int, []),
    ('dkv_last_error', ctypes.c_char_p, []),
    ('dkv_subblock_bytes', ctypes.c_int64, [ctypes.c_int32, ctypes.c_int32]),
    ('dkv_slab_bytes', ctypes.c_int64, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    ('dkv_pack', ctypes.c_int, [ctypes.POINTER(PackJob), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_pack_batch', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                      ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_void_p]),
    ('dkv_pack_validate', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                         ctypes.c_int32]),
    ('dkv_reconstruct', ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                       ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_attend_workspace_bytes', ctypes.c_int64, [ctypes.POINTER(AttnArgs)]),
    ('dkv_attend', ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    ('dkv_attend_noalloc', ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    ('dkv_export', ctypes.c_int, [ctypes.POINTER(SegmentIO), ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                  ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_import', ctypes.c_int, [ctypes.POINTER(SegmentIO), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                  ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_segment_batch', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                         ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_segment_validate', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                            ctypes.c_int32, ctypes.c_int32]),
    ('dkv_rope_qkv', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    ('dkv_rope_pack', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.c_void_p]),
    ('dkv_linear_supported', ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.c_int32]),
    ('dkv_linear', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                  ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_float, ctypes.c_int32,
                                  ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]),
    ('dkv_linear_tiled', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                        ctypes.c_float, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]),
    ('dkv_rms_norm', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p]),
    ('dkv_silu_mul', ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]),
]


def lib_path():
    return _build.LIB_PATH


def load():
    """Loads libdkv.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(f'{path} is missing: build it first (python -c "import __graft_entry__ as g; g.build()")')
    lib = ctypes.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.dkv_version() != ABI_VERSION:
        raise RuntimeError(f'libdkv ABI {lib.dkv_version()} != expected {ABI_VERSION}')
    _lib = lib
    return lib


def check(rc, what):
    """Turns a C status into the reference's exception types."""
    if rc == 0:
        return
    if rc == DKV_EINVAL:
        raise ValueError(load().dkv_last_error().decode() or f'{what}: invalid argument')
    raise RuntimeError(f'{what}: HIP error {rc}')


_raw_stream = getattr(torch._C, '_cuda_getCurrentRawStream', None)


def stream_handle(device=None):
    """torch's current stream on `device` (a torch.device, an index or None: the current device) as
    a hipStream_t. Every launch asks: the current stream changes under torch.cuda.stream() and
    during graph capture."""
    if _raw_stream is not None:
        if isinstance(device, str):
            device = torch.device(device)
        index = device.index if isinstance(device, torch.device) else device
        return ctypes.c_void_p(_raw_stream(torch.cuda.current_device() if index is None else index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def subblock_bytes(rows, bits):
    return load().dkv_subblock_bytes(rows, bits)


def slab_bytes(rows, bits, layers, heads):
    return load().dkv_slab_bytes(rows, bits, layers, heads)
