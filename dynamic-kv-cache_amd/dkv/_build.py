"""Builds libdkv.so (the HIP kernels and their C ABI) for gfx950 with hipcc.

Flags that matter for results:
  -ffp-contract=off                          no silent FMA contraction: the
                                             pack arithmetic and the q*s + a
                                             dequantization round like the
                                             reference's separate torch ops
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE fp32 division in the pack
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no packed fp32 VALU instructions
"""
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)  # dynamic-kv-cache_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, 'csrc')
INCLUDE = os.path.join(REPO, 'include')
LIB_NAME = 'libdkv.so'
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# The timeline build (-DDKV_TIMELINE): the attention kernels also record per-workgroup
# wall-clock stamps that dkv_timeline_short / dkv_timeline_mfma copy out. A diagnostic library,
# never the one the package loads unless bench.py --timeline points it there.
TIMELINE_LIB_PATH = os.path.join(PKG_DIR, 'libdkv_timeline.so')
# The in-kernel merge build (-DDKV_INKERNEL_MERGE=1): the frame-chunk kernel merges its own history
# splits (the last workgroup of each KV head) instead of a second launch. A measurement build for
# bench.py --lib, slower than the library's two launches at every shape timed.
INKERNEL_LIB_PATH = os.path.join(PKG_DIR, 'libdkv_inkernel_merge.so')
INKERNEL_TIMELINE_LIB_PATH = os.path.join(PKG_DIR, 'libdkv_inkernel_merge_timeline.so')
ARCH = os.environ.get('DKV_OFFLOAD_ARCH', 'gfx950')

HIPCC_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-shared',
    '-ffp-contract=off', '-fhip-fp32-correctly-rounded-divide-sqrt',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-command-line-argument',
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith('.hip'))


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found: libdkv needs ROCm to build')
    return path


def build(verbose=False, extra=(), out=None):
    """Compiles every csrc/*.hip into one shared library next to this file (or at `out`)."""
    out = out or LIB_PATH
    tmp = out + '.tmp'
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, '-I', INCLUDE, '-I', CSRC, '-o', tmp, *sources()]
    if verbose:
        print(' '.join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f'hipcc failed with status {proc.returncode}')
    os.replace(tmp, out)
    return out


if __name__ == '__main__':
    timeline, inkernel = '--timeline' in sys.argv[1:], '--in-kernel-merge' in sys.argv[1:]
    extra = (['-DDKV_TIMELINE'] if timeline else []) + (['-DDKV_INKERNEL_MERGE=1'] if inkernel else [])
    out = {(False, False): LIB_PATH, (True, False): TIMELINE_LIB_PATH, (False, True): INKERNEL_LIB_PATH,
           (True, True): INKERNEL_TIMELINE_LIB_PATH}[(timeline, inkernel)]
    print(build(verbose=True, extra=extra, out=out))
