"""Build libtreeattn.so (gfx950) in-tree with hipcc.

    python -m treeattn_amd.build            # compile every source, link the library
    python -m treeattn_amd.build --trace attend.hip   # a tracing build of one source (treeattn_amd.phase_trace)

Every HIP source is compiled for gfx950 only, with packed-fp32 instruction generation disabled.  The
selection kernels (select.hip) are compiled with floating-point contraction off so their scores follow
the canonical float32 order exactly.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
OBJ = os.path.join(HERE, '_build')
LIB = os.path.join(HERE, 'libtreeattn.so')
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')

SOURCES = {
    'abi.hip': [],
    'cand.hip': [],
    'select.hip': ['-ffp-contract=off'],
    'attend.hip': [],
    'attend_static.hip': [],
    'attend_bwd.hip': [],
    'sample.hip': [],
    'gemm.hip': [],
    'rowmm_nt.hip': [],
    'rowvec.hip': [],
    'gather_blocks.hip': [],
    'prefill_attn.hip': [],
    'step.hip': [],
    'calib.hip': [],
    'neighbor.hip': [],
    'gate.hip': [],
    'forest.hip': [],
    'lanetree.hip': [],
}

COMMON = ['--offload-arch=gfx950', '-O3', '-fPIC', '-std=c++17', '-Wall', '-Wno-unused-function',
          '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
          '-I', os.path.join(HERE, '..', 'include')]


def _compile(name):
    src = os.path.join(CSRC, name)
    obj = os.path.join(OBJ, name.replace('.hip', '.o'))
    cmd = [HIPCC, '-c', src, '-o', obj] + COMMON + SOURCES[name]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('hipcc failed for %s:\n%s\n%s' % (name, ' '.join(cmd), r.stderr[-6000:]))
    return obj


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, sorted(SOURCES)))
    tmp = LIB + '.tmp'
    cmd = [HIPCC, '-shared', '-fPIC', '--offload-arch=gfx950', '-o', tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('link failed:\n%s' % r.stderr[-4000:])
    os.replace(tmp, LIB)
    if verbose:
        print('built', LIB)
    return LIB


def trace_lib_path(name):
    """Path of the tracing build of source `name` (see build_trace)."""
    return os.path.join(HERE, 'libtreeattn_trace_%s.so' % name.replace('.hip', ''))


def build_trace(name, verbose=True):
    """A tracing build: source `name` (one of SOURCES) compiled with -DTA_TRACE, so that its phase marks store
    time stamps (csrc/trace.hpp), and linked with the library's other objects (from a previous build()) into
    libtreeattn_trace_<name>.so beside the library.  treeattn_amd.phase_trace loads it."""
    if name not in SOURCES:
        raise ValueError('unknown source %s' % name)
    os.makedirs(OBJ, exist_ok=True)
    src = os.path.join(CSRC, name)
    obj = os.path.join(OBJ, 'trace_' + name.replace('.hip', '.o'))
    cmd = [HIPCC, '-c', src, '-o', obj] + COMMON + SOURCES[name] + ['-DTA_TRACE']
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('hipcc failed for %s (tracing):\n%s' % (name, r.stderr[-6000:]))
    objs = [os.path.join(OBJ, n.replace('.hip', '.o')) for n in sorted(SOURCES) if n != name]
    missing = [o for o in objs if not os.path.exists(o)]
    if missing:
        raise RuntimeError('run python -m treeattn_amd.build first (missing %s)' % ', '.join(missing))
    lib = trace_lib_path(name)
    r = subprocess.run([HIPCC, '-shared', '-fPIC', '--offload-arch=gfx950', '-o', lib + '.tmp'] + objs + [obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('link failed:\n%s' % r.stderr[-4000:])
    os.replace(lib + '.tmp', lib)
    if verbose:
        print('built', lib)
    return lib


if __name__ == '__main__':
    if len(sys.argv) > 2 and sys.argv[1] == '--trace':
        build_trace(sys.argv[2])
    else:
        build()
    sys.exit(0)
