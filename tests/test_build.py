"""Build-level guards for the gfx950 kernels (CPU only: hipcc cross-compiles).

Every kernel must run without scratch (private) memory: a spill or a local copy of the
by-value argument block turns register accesses into memory round trips. Checked from hipcc's
kernel-resource-usage remarks with the library's own flags.
"""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from dkv import _build

HIPCC = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'


@pytest.mark.skipif(not os.path.exists(HIPCC), reason='hipcc not installed')
def test_every_kernel_runs_without_scratch(tmp_path):
    flags = [f for f in _build.HIPCC_FLAGS if f not in ('-shared', '-fPIC')]

    def remarks(src):
        out = tmp_path / (os.path.basename(src) + '.o')
        cmd = [HIPCC, *flags, '--cuda-device-only', '-c', '-I', _build.INCLUDE, '-I', _build.CSRC, src, '-o', str(out),
               '-Rpass-analysis=kernel-resource-usage']
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        return proc.stderr

    with ThreadPoolExecutor(max_workers=4) as pool:
        logs = list(pool.map(remarks, _build.sources()))
    kernels = 0
    for log in logs:
        names = re.findall(r'Function Name: (\S+)', log)
        scratch = [int(x) for x in re.findall(r'ScratchSize \[bytes/lane\]: (\d+)', log)]
        assert len(names) == len(scratch)
        kernels += len(names)
        for name, size in zip(names, scratch):
            assert size == 0, f'{name} uses {size} bytes/lane of scratch'
    assert kernels >= 10
