"""Builds the gfx950 device library and the protocol server in-tree.

    python -m cpde_amd.build            # both
    python -m cpde_amd.build lib        # libcpde_hip.so only

Outputs: cpde_amd/lib/libcpde_hip.so and cpde_amd/bin/cpde_server (rpath to
../lib).  Every HIP translation unit is compiled for gfx950 with packed-FP32
instruction selection disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / 'csrc'
LIB_DIR = PKG / 'lib'
BIN_DIR = PKG / 'bin'
LIB = LIB_DIR / 'libcpde_hip.so'
SERVER = BIN_DIR / 'cpde_server'
ARCH = os.environ.get('CPDE_OFFLOAD_ARCH', 'gfx950')
HIP_FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
             '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
             '-Wno-unused-command-line-argument']


def hipcc():
    exe = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(exe).exists():
        raise RuntimeError('hipcc not found; the device library needs ROCm')
    return exe


def _run(cmd):
    print(' '.join(str(c) for c in cmd), flush=True)
    subprocess.run([str(c) for c in cmd], check=True)


def build_lib():
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = PKG / '_build'
    obj_dir.mkdir(exist_ok=True)
    # the layer-fused kernel templates are compiled at run time (hipRTC, per
    # schema); embed their text into the library
    text = (CSRC / 'fused.hip.in').read_text()
    assert ')CPDE_SRC"' not in text
    embedded = obj_dir / 'fused_source.cpp'
    embedded.write_text('namespace cpde {\nextern const char* const kFusedSource;\n'
                        'const char* const kFusedSource = R"CPDE_SRC(' + text + ')CPDE_SRC";\n}\n')
    objs = []
    for src in [CSRC / 'kernels.hip', CSRC / 'api.hip', CSRC / 'tables.cpp', CSRC / 'jit.cpp', embedded]:
        obj = obj_dir / (src.name + '.o')
        _run([hipcc(), *HIP_FLAGS, '-I', ROOT / 'include', '-c', src, '-o', obj])
        objs.append(obj)
    tmp = LIB.with_suffix('.so.tmp')
    _run([hipcc(), *HIP_FLAGS, '-shared', '-o', tmp, *objs, '-lhiprtc'])
    os.replace(tmp, LIB)
    return LIB


def build_server():
    if not (CSRC / 'server.cpp').exists():
        return None
    BIN_DIR.mkdir(exist_ok=True)
    tmp = SERVER.with_name('cpde_server.tmp')
    _run(['g++', '-O2', '-std=c++17', '-pthread', '-I', ROOT / 'include', '-I', '/opt/rocm/include',
          CSRC / 'server.cpp', '-o', tmp, '-L', LIB_DIR, '-lcpde_hip', '-Wl,-rpath,$ORIGIN/../lib'])
    os.replace(tmp, SERVER)
    return SERVER


def warm_jit():
    """Compile the schema-specialised kernels of the benchmark workloads into
    the code-object cache (cpde_amd/jit_cache), so that a fresh process on the
    GPU finds them without compiling."""
    from . import hip, workloads as W
    cache = PKG / 'jit_cache'
    if cache.exists():
        shutil.rmtree(cache)
    hip.load(LIB)
    for table, neurons, width in [(W.full_schema(2, 6), [2, 128, 128, 128, 128, 1], 729),
                                  (W.full_schema(2, 2), [2, 128, 128, 128, 128, 1], 729),
                                  (W.full_schema(3, 4), [3, 128, 128, 128, 128, 128, 1], 32768),
                                  (W.full_schema(2, 6), [2, 256, 256, 256, 256, 1], 65536),
                                  (W.closed_schema(2, [(2, 0), (0, 2)]), [2, 64, 64, 64, 1], 4096),
                                  (W.closed_schema(2, []), [2, 64, 64, 64, 1], 256),
                                  (W.full_schema(2, 6), [2, 32, 32, 1], 40)]:  # __graft_entry__.smoke
        hip.jit_prepare(table, neurons, width, 256, ARCH)


def main(argv):
    what = argv[1] if len(argv) > 1 else 'all'
    if what in ('all', 'lib'):
        build_lib()
        warm_jit()
    if what in ('all', 'server'):
        build_server()


if __name__ == '__main__':
    main(sys.argv)
