"""The C ABI on the CPU: the library loads, exports what include/dkv.h declares, its struct
layouts match the ctypes mirror, and invalid arguments fail before any device work."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import REPO
from dkv import _lib
from dkv.gpu_cache import segment_bytes, slab_bytes, subblock_bytes

HEADER = os.path.join(REPO, 'include', 'dkv.h')


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'^\s*(?:int|int64_t|const char\*)\s+(dkv_\w+)\s*\(', text, re.M)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
    assert {n for n, _, _ in _lib.SIGNATURES} == set(names)
    assert lib.dkv_version() == _lib.ABI_VERSION == 3


STRUCT_PROBE = r'''
#include <stdio.h>
#include <stddef.h>
#include "dkv.h"
#define F(s, f) printf(#s " " #f " %zu\n", offsetof(s, f));
int main(void) {
  printf("dkv_tile size %zu\n", sizeof(dkv_tile));
  printf("dkv_pack_job size %zu\n", sizeof(dkv_pack_job));
  printf("dkv_attn_args size %zu\n", sizeof(dkv_attn_args));
  printf("dkv_segment_io size %zu\n", sizeof(dkv_segment_io));
  printf("DKV_MAX_CHUNK_SEGS const %d\n", DKV_MAX_CHUNK_SEGS);
  printf("DKV_NOALLOC_SCRATCH_BYTES const %d\n", DKV_NOALLOC_SCRATCH_BYTES);
  printf("DKV_ABI_VERSION const %d\n", DKV_ABI_VERSION);
  printf("DKV_ARG_TILES const %d\n", DKV_ARG_TILES);
  %FIELDS%
  return 0;
}
'''


@pytest.mark.parametrize('cls,cname', [(_lib.Tile, 'dkv_tile'), (_lib.PackJob, 'dkv_pack_job'),
                                       (_lib.AttnArgs, 'dkv_attn_args'), (_lib.SegmentIO, 'dkv_segment_io')])
def test_struct_layout_matches_header(tmp_path, cls, cname):
    fields = '\n'.join(f'F({cname}, {f})' for f, _ in cls._fields_)
    src = tmp_path / 'probe.c'
    src.write_text(STRUCT_PROBE.replace('%FIELDS%', fields))
    exe = tmp_path / 'probe'
    subprocess.run(['gcc', '-std=c11', '-I', os.path.dirname(HEADER), str(src), '-o', str(exe)], check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split('\n')
    sizes = {l.split()[0]: int(l.split()[2]) for l in lines if ' size ' in l}
    assert sizes[cname] == ctypes.sizeof(cls)
    consts = {l.split()[0]: int(l.split()[2]) for l in lines if ' const ' in l}
    assert consts == dict(DKV_MAX_CHUNK_SEGS=_lib.DKV_MAX_CHUNK_SEGS,
                          DKV_NOALLOC_SCRATCH_BYTES=_lib.DKV_NOALLOC_SCRATCH_BYTES, DKV_ABI_VERSION=_lib.ABI_VERSION,
                          DKV_ARG_TILES=_lib.DKV_ARG_TILES)
    for line in lines:
        parts = line.split()
        if len(parts) == 3 and parts[0] == cname and parts[1] != 'size':
            assert getattr(cls, parts[1]).offset == int(parts[2]), parts[1]


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_geometry_matches_python_mirror(bits):
    for rows in range(1, 65):
        assert _lib.subblock_bytes(rows, bits) == subblock_bytes(rows, bits)
        assert _lib.slab_bytes(rows, bits, 32, 5) == slab_bytes(rows, bits, 32, 5)
        assert subblock_bytes(rows, bits) % 16 == 0
    assert subblock_bytes(64, bits) == 64 * {4: 40, 8: 72, 16: 128}[bits]
    assert segment_bytes(150, bits, 2, 5) == 2 * slab_bytes(64, bits, 2, 5) + slab_bytes(22, bits, 2, 5)


def job(**kw):
    base = dict(k=16, v=16, k_head_stride=64, k_tok_stride=64 * 5, v_head_stride=64, v_tok_stride=64,
                seg_offset=0, seg_rows=64, seg_token_start=0, row0=0, n=8, layer=0, bits=4,
                tile_index0=0, write_tiles=0)
    base.update(kw)
    return _lib.PackJob(**base)


@pytest.mark.parametrize('kw,msg', [
    (dict(bits=5), 'bits'),
    (dict(row0=60), 'outside a segment'),
    (dict(layer=3), 'layer'),
    (dict(seg_offset=8), 'misaligned'),
    (dict(k=18), 'aligned'),
    (dict(v_tok_stride=63), 'aligned'),
])
def test_pack_rejects_bad_jobs_without_touching_the_device(kw, msg):
    lib = _lib.load()
    j = job(**kw)
    rc = lib.dkv_pack(ctypes.byref(j), ctypes.c_void_p(4096), 1 << 20, None, 2, 5, None)
    assert rc == _lib.DKV_EINVAL
    assert msg in lib.dkv_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(rc, 'dkv_pack')


def test_pack_rejects_segment_past_arena_end():
    lib = _lib.load()
    j = job(seg_offset=1 << 20)
    assert lib.dkv_pack(ctypes.byref(j), ctypes.c_void_p(4096), 1 << 20, None, 2, 5, None) == _lib.DKV_EINVAL


def attn(**kw):
    a = _lib.AttnArgs()
    a.q = a.k_new = a.v_new = a.out = 4096
    a.q_head_stride, a.q_tok_stride = 64 * 64, 64
    a.kn_head_stride, a.kn_tok_stride = 64 * 64, 64
    a.vn_head_stride, a.vn_tok_stride = 64 * 64, 64
    a.layers, a.heads, a.q_heads, a.nq = 1, 5, 15, 64
    a.out_tok_stride, a.out_head_stride = 15 * 64, 64
    a.scale = 0.125
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize('kw,msg', [
    (dict(q=0), 'null'),
    (dict(q_heads=14), 'shape'),
    (dict(n_segs=17), 'n_segs'),
    (dict(out_dtype=2), 'out_dtype'),
    (dict(q_tok_stride=60), 'aligned'),
    (dict(n_tiles=3), 'null'),
    (dict(out=4096 + 8), 'out must be'),
    (dict(out_tok_stride=15 * 64 + 2), 'out must be'),
])
def test_attend_rejects_bad_arguments(kw, msg):
    lib = _lib.load()
    a = attn(**kw)
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL
    assert msg in lib.dkv_last_error().decode()


def test_attend_rejects_bad_segments():
    lib = _lib.load()
    a = attn(n_segs=2)
    a.seg_bounds[0], a.seg_bounds[1], a.seg_bounds[2] = 0, 70, 64
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL
    a.seg_bounds[1] = 0
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL


def host_tiles(rows):
    """A dkv_tile array of consecutive tiles of the given row counts (8-bit, packed one after
    another)."""
    arr = (_lib.Tile * len(rows))()
    start = 0
    for i, r in enumerate(rows):
        arr[i].offset, arr[i].token_start, arr[i].rows, arr[i].bits = 4096 * i, start, r, 8
        start += r
    return arr


@pytest.mark.parametrize('change', [None, 'bits', 'rows', 'gap', 'short', 'step'])
def test_attend_checks_the_host_tile_copy(change):
    """tiles_host (the descriptors the frame-chunk kernel then takes from its argument block) must
    be well formed and cover [0, past) in token order; a bad copy is refused before any launch.
    With a device step pair the copy is not used and not checked."""
    lib = _lib.load()
    arr = host_tiles([64, 64, 30])
    a = attn(past=158, n_tiles=3, arena=4096, tiles=4096)
    if change == 'bits':
        arr[1].bits = 5
    elif change == 'rows':
        arr[2].rows = 65
    elif change == 'gap':
        arr[2].token_start = 129
    elif change == 'short':
        a.past = 159  # the tiles end at 158
    elif change == 'step':
        arr[1].bits = 5
        a.step = 4096
    a.tiles_host = ctypes.addressof(arr)
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL
    msg = lib.dkv_last_error().decode()
    if change in (None, 'step'):
        assert 'workspace' in msg  # past the tile checks, at the next one
    else:
        assert 'tiles_host' in msg, msg


def test_attend_demands_workspace_when_split():
    lib = _lib.load()
    a = attn(past=4096, n_tiles=64, arena=4096, tiles=4096)
    need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
    assert need > 0
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL
    assert 'workspace' in lib.dkv_last_error().decode()


def test_attend_workspace_matches_the_partial_format():
    """Per split row: 64 fp16 O / sum values + (max, sum) in bf16 precision, 64 fp32 O + (max, sum)
    in fp32 precision; the short-chunk kernel (path 3) keeps fp32 rows in both precisions, one
    split per 4 units (64-token tiles plus the chunk) by default, at most 64 per KV head. Auto
    takes the frame-chunk kernel for decode steps too: in bf16 precision its 4-wave variant, four
    workgroups per CU, so one unit per split up to that cap (4 x 256 CUs / 5 KV heads without a
    device); in fp32 precision, and with path 2, the 12-wave kernel, one workgroup per CU. One
    split needs no workspace."""
    lib = _lib.load()
    need = {}
    for precision in (0, 1):
        a = attn(past=4096, n_tiles=64, arena=4096, tiles=4096, precision=precision)
        need[precision] = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
    rows = need[1] // (64 * 4 + 8)
    assert rows > 0 and need[1] == rows * (64 * 4 + 8) and need[0] == rows * (64 * 2 + 8)
    for precision in (0, 1):
        a = attn(past=4096, n_tiles=64, arena=4096, tiles=4096, nq=1, precision=precision, path=3)
        splits = (64 + 1 + 3) // 4
        assert lib.dkv_attend_workspace_bytes(ctypes.byref(a)) == a.heads * splits * 3 * (64 * 4 + 8)
        long = attn(past=64 * 600, n_tiles=600, arena=4096, tiles=4096, nq=1, precision=precision, path=3)
        assert lib.dkv_attend_workspace_bytes(ctypes.byref(long)) == long.heads * 64 * 3 * (64 * 4 + 8)
        one = attn(past=4096, n_tiles=64, arena=4096, tiles=4096, nq=1, precision=precision, splits=1)
        assert lib.dkv_attend_workspace_bytes(ctypes.byref(one)) == 0
        auto = attn(past=4096, n_tiles=64, arena=4096, tiles=4096, nq=1, precision=precision)
        mfma = attn(past=4096, n_tiles=64, arena=4096, tiles=4096, nq=1, precision=precision, path=2)
        units = 64 + 1
        row = 64 * (4 if precision else 2) + 8  # fp32 O or fp16 O / sum, then (max, sum)
        per = (units + 51 - 1) // 51  # 12 waves: one workgroup per CU, cap 256 // 5 = 51
        big = mfma.heads * ((units + per - 1) // per) * 3 * row
        assert lib.dkv_attend_workspace_bytes(ctypes.byref(mfma)) == big
        # auto: bf16 one split per unit (65 <= 204), 3 query rows each; fp32 as path 2
        assert lib.dkv_attend_workspace_bytes(ctypes.byref(auto)) == (auto.heads * units * 3 * row if precision == 0 else big)


def test_pack_validate_checks_every_job_of_a_host_table():
    lib = _lib.load()
    good = [job(seg_offset=0), job(seg_offset=4096, layer=1)]
    table = (_lib.PackJob * 2)(*good)
    assert lib.dkv_pack_validate(ctypes.addressof(table), 2, 1 << 20, 2, 5) == 0
    bad = (_lib.PackJob * 3)(*good, job(seg_offset=1 << 20))
    assert lib.dkv_pack_validate(ctypes.addressof(bad), 3, 1 << 20, 2, 5) == _lib.DKV_EINVAL
    assert 'outside' in lib.dkv_last_error().decode()
    neg = (_lib.PackJob * 1)(job(write_tiles=1, tile_index0=-1))
    assert lib.dkv_pack_validate(ctypes.addressof(neg), 1, 1 << 20, 2, 5) == _lib.DKV_EINVAL


@pytest.mark.parametrize('kw', [dict(path=3), dict(path=-1), dict(precision=2)])
def test_attend_rejects_unknown_path_or_precision(kw):
    lib = _lib.load()
    a = attn(**kw)
    assert lib.dkv_attend(ctypes.byref(a), None) == _lib.DKV_EINVAL
    assert 'path' in lib.dkv_last_error().decode()


def seg_io(**kw):
    s = _lib.SegmentIO()
    s.payload[0], s.payload[1] = 4096, 8192
    s.offsets[0], s.offsets[1], s.scales[0], s.scales[1] = 4096, 4100, 4104, 4108
    s.seg_offset, s.seg_rows, s.seg_token_start, s.row0, s.rows, s.bits = 0, 64, 0, 0, 64, 4
    s.layer0, s.n_layers, s.tile_index0, s.write_tiles = 0, 2, 0, 0
    for k, v in kw.items():
        setattr(s, k, v)
    return s


@pytest.mark.parametrize('kw,msg', [
    (dict(bits=2), 'bits'),
    (dict(n_layers=3), 'layers'),
    (dict(layer0=-1), 'layers'),
    (dict(row0=10, rows=60), 'outside a segment'),
    (dict(seg_offset=1 << 20), 'outside'),
    (dict(seg_offset=24), 'misaligned'),
    (dict(offsets=(ctypes.c_void_p * 2)(0, 0)), 'offset and scale'),
])
def test_segment_io_rejects_bad_segments_without_touching_the_device(kw, msg):
    lib = _lib.load()
    s = seg_io(**kw)
    assert lib.dkv_export(ctypes.byref(s), ctypes.c_void_p(4096), 1 << 20, 2, 5, None) == _lib.DKV_EINVAL
    assert msg in lib.dkv_last_error().decode()
    assert lib.dkv_import(ctypes.byref(s), ctypes.c_void_p(4096), 1 << 20, ctypes.c_void_p(4096), 2, 5,
                          None) == _lib.DKV_EINVAL
    table = (_lib.SegmentIO * 2)(seg_io(), s)
    assert lib.dkv_segment_validate(ctypes.addressof(table), 2, 0, 1 << 20, 2, 5) == _lib.DKV_EINVAL


def test_segment_io_payload_alignment_and_tile_table():
    lib = _lib.load()
    s = seg_io()
    s.payload[1] = 8200
    assert lib.dkv_export(ctypes.byref(s), ctypes.c_void_p(4096), 1 << 20, 2, 5, None) == _lib.DKV_EINVAL
    assert '16-byte' in lib.dkv_last_error().decode()
    t = seg_io(write_tiles=1)
    assert lib.dkv_import(ctypes.byref(t), ctypes.c_void_p(4096), 1 << 20, None, 2, 5, None) == _lib.DKV_EINVAL
    assert 'tile table' in lib.dkv_last_error().decode()
    sixteen = seg_io(bits=16, offsets=(ctypes.c_void_p * 2)(0, 0), scales=(ctypes.c_void_p * 2)(0, 0))
    table = (_lib.SegmentIO * 2)(seg_io(), sixteen)
    assert lib.dkv_segment_validate(ctypes.addressof(table), 2, 1, 1 << 20, 2, 5) == 0
    neg = (_lib.SegmentIO * 1)(seg_io(write_tiles=1, tile_index0=-1))
    assert lib.dkv_segment_validate(ctypes.addressof(neg), 1, 1, 1 << 20, 2, 5) == _lib.DKV_EINVAL
    assert lib.dkv_segment_batch(ctypes.addressof(table), 2, 64, 2, 2, ctypes.c_void_p(4096), 1 << 20, None, 2, 5,
                                 None) == _lib.DKV_EINVAL


def test_pointwise_ops_reject_misaligned_buffers():
    lib = _lib.load()
    ok = ctypes.c_void_p(4096)
    bad = ctypes.c_void_p(4098)
    assert lib.dkv_rope_qkv(bad, 1600, ok, ok, 64, 4, 15, 5, ok, ok, ok, None) == _lib.DKV_EINVAL
    assert lib.dkv_rope_qkv(ok, 1000, ok, ok, 64, 4, 15, 5, ok, ok, ok, None) == _lib.DKV_EINVAL  # row too short
    assert lib.dkv_rms_norm(ok, 960, ok, ok, 960, 4, 12, 1e-5, None) == _lib.DKV_EINVAL  # dim % 8
    assert lib.dkv_rms_norm(ok, 964, ok, ok, 960, 4, 960, 1e-5, None) == _lib.DKV_EINVAL  # stride % 8
    assert lib.dkv_silu_mul(ok, 5120, bad, 2560, 4, 2560, None) == _lib.DKV_EINVAL
    assert lib.dkv_silu_mul(ok, 4000, ok, 2560, 4, 2560, None) == _lib.DKV_EINVAL  # row holds < 2 * inter
    assert 'dkv_silu_mul' in lib.dkv_last_error().decode()
    assert lib.dkv_rms_norm(ok, 960, ok, ok, 960, 0, 960, 1e-5, None) == 0  # no rows: nothing to launch


def test_rope_pack_rejects_bad_arguments_without_touching_the_device():
    lib = _lib.load()
    ok, bad = ctypes.c_void_p(4096), ctypes.c_void_p(4098)
    arena = ctypes.c_void_p(1 << 16)

    def call(qkv=ok, stride=1600, n=64, j=None, on_device=0):
        j = job(n=64) if j is None else j
        return lib.dkv_rope_pack(qkv, stride, ok, ok, 64, n, 15, ok, ok, ok, ctypes.byref(j), on_device, arena,
                                 1 << 20, ok, 2, 5, None)

    assert call(qkv=bad) == _lib.DKV_EINVAL
    assert call(stride=1000) == _lib.DKV_EINVAL  # a row holds fewer than 25 heads
    assert call(n=32) == _lib.DKV_EINVAL and 'projection holds' in lib.dkv_last_error().decode()
    assert call(j=job(n=64, bits=5)) == _lib.DKV_EINVAL and 'bits' in lib.dkv_last_error().decode()
    assert call(n=0, on_device=1) == _lib.DKV_EINVAL and 'device job' in lib.dkv_last_error().decode()
    assert lib.dkv_rope_pack(ok, 1600, ok, ok, 64, 64, 15, ok, ok, ok, None, 0, arena, 1 << 20, ok, 2, 5,
                             None) == _lib.DKV_EINVAL  # no job


def test_linear_rejects_unsupported_shapes_without_touching_the_device():
    lib = _lib.load()
    ok = ctypes.c_void_p(4096)
    assert lib.dkv_linear_supported(64, 1600, 960, 1, 0) == 1
    assert lib.dkv_linear_supported(64, 5120, 960, 1, 2) == 1
    assert lib.dkv_linear_supported(100, 960, 2560, 0, 1) == 1
    assert lib.dkv_linear_supported(64, 960, 900, 0, 0) == 0  # k % 64
    assert lib.dkv_linear_supported(64, 1000, 960, 0, 0) == 0  # n % 16
    assert lib.dkv_linear_supported(64, 960, 2048, 1, 0) == 0  # norm needs k <= 1024
    assert lib.dkv_linear_supported(64, 960, 960, 0, 3) == 0  # no such epilogue
    assert lib.dkv_linear(ok, 960, ok, 960, 64, 960, 900, None, 1e-5, 0, None, 0, ok, 960, None) == _lib.DKV_EINVAL
    assert 'dkv_linear' in lib.dkv_last_error().decode()
    assert lib.dkv_linear(ok, 960, ok, 960, 64, 960, 960, None, 1e-5, 1, None, 0, ok, 960,
                          None) == _lib.DKV_EINVAL  # residual epilogue without a residual
    assert lib.dkv_linear(ctypes.c_void_p(4098), 960, ok, 960, 64, 960, 960, None, 1e-5, 0, None, 0, ok, 960,
                          None) == _lib.DKV_EINVAL  # misaligned x
    assert lib.dkv_linear(ok, 960, ok, 960, 0, 960, 960, None, 1e-5, 0, None, 0, ok, 960, None) == 0  # no rows
    # dkv_linear_tiled: undefined layout bits, a tiled out whose n_out is not a multiple of 64
    assert lib.dkv_linear_tiled(ok, 960, ok, 960, 64, 960, 960, None, 1e-5, 0, None, 0, ok, 960, 16,
                                None) == _lib.DKV_EINVAL
    # a tiled residual needs the residual epilogue
    assert lib.dkv_linear_tiled(ok, 960, ok, 960, 64, 960, 960, None, 1e-5, 0, None, 0, ok, 960, 8,
                                None) == _lib.DKV_EINVAL
    assert lib.dkv_linear_tiled(ok, 960, ok, 960, 64, 976, 960, None, 1e-5, 0, None, 0, ok, 976, 4,
                                None) == _lib.DKV_EINVAL
    assert 'layout' in lib.dkv_last_error().decode()
    # row strides of tiled operands are not checked
    assert lib.dkv_linear_tiled(ok, 0, ok, 0, 0, 960, 960, None, 1e-5, 0, None, 0, ok, 0, 7, None) == 0
    assert lib.dkv_linear_tiled(ok, 0, ok, 0, 0, 960, 960, None, 1e-5, 1, ok, 0, ok, 0, 15, None) == 0
