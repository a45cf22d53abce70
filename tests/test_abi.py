"""The C ABI library loads, exports every entry point include/bvml_dsine.h
declares, and rejects bad arguments before touching the GPU (all calls here
fail validation, so none launches; the runs need no device).  Also runs the
C++ drop-in's error-path test (tests/cpp, cpu mode)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from brovisionml_amd import _lib
from brovisionml_amd.build import LIB, ROOT

HEADER = os.path.join(ROOT, "include", "bvml_dsine.h")
CPP_TEST = os.path.join(ROOT, "tests", "cpp", "_build", "test_dsine_ops")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:long\s+)?\w+\s*\*?\s*(bvml_dsine_\w+)\s*\(",
                                 text, re.M)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_heads_pack_host_checks():
    """bvml_dsine_heads_pack_f32 and _packed_size run on the host: sizes and
    argument checks (the packed layout itself is checked on the GPU through
    the kernel, tests/test_gpu_heads.py)."""
    lib = _lib.load()
    assert lib.bvml_dsine_heads_packed_size(25) == 2 * 1024
    assert lib.bvml_dsine_heads_packed_size(576) == 36 * 1024
    assert lib.bvml_dsine_heads_packed_size(0) == -1
    assert lib.bvml_dsine_heads_packed_size(4097) == -1
    import numpy as np
    w2p, w4p = _lib.heads_pack_f32(np.ones((2, 64, 64), np.float32),
                                   [np.ones((17, 64), np.float32), np.ones((1, 64), np.float32)])
    assert w2p.shape == (8192,) and (w2p == 1).all()
    # the first output block of the 17-output head holds 16 real rows, the
    # second 1 real row and 15 zero rows
    assert w4p[0].shape == (2048,) and w4p[0].sum() == 17 * 64
    assert w4p[1].sum() == 64
    vp = ctypes.c_void_p
    outs = (ctypes.c_int * 1)(25)
    assert lib.bvml_dsine_heads_pack_f32(None, (vp * 1)(), outs, 1, None, (vp * 1)()) == _lib.ENULL
    assert lib.bvml_dsine_heads_pack_f32(None, None, outs, 0, None, None) == _lib.EPARAM


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}\b", out), name


def test_version():
    assert _lib.load().bvml_dsine_version().decode() == "0.2.0"


FAKE = 0x10000  # never dereferenced: validation fails or the call is a no-op first


def angmf(**kw):
    args = dict(pred_norm=FAKE, prob=FAKE + 0x100000, xy=FAKE + 0x200000, angle=FAKE + 0x300000,
                ray=FAKE + 0x400000, fu=100.0, cu=10.0, fv=100.0, cv=10.0, B=1, H=4, W=4, k=5,
                ray_bstride=0, out=FAKE + 0x500000, flags=0, stream=0)
    args.update(kw)
    return _lib.angmf_propagate_f32(**args)


@pytest.mark.parametrize("kw,code", [
    (dict(B=-1), _lib.ESHAPE), (dict(H=-2), _lib.ESHAPE), (dict(ray_bstride=-3), _lib.ESHAPE),
    (dict(k=4), _lib.EK), (dict(k=11), _lib.EK), (dict(k=0), _lib.EK),
    (dict(prob=0), _lib.ENULL), (dict(out=0), _lib.ENULL),
    (dict(flags=8), _lib.EFLAGS),
    (dict(out=FAKE), _lib.EALIAS),                  # out == pred_norm
    (dict(out=FAKE + 0x200000 + 64), _lib.EALIAS),  # inside xy
    (dict(H=1 << 16, W=1 << 14), _lib.ESIZE),       # plane of 2^30 pixels
])
def test_angmf_rejects(kw, code):
    assert angmf(**kw) == code
    assert _lib.last_error().startswith("angmf_propagate: ")


def test_angmf_ray_from_intrinsics_validation():
    # with the flag the ray pointer may be NULL; the other checks still apply
    synth = _lib.RAY_FROM_INTRINSICS
    assert angmf(flags=synth, ray=0, B=-1) == _lib.ESHAPE
    assert angmf(flags=synth, ray=0, prob=0) == _lib.ENULL
    assert angmf(flags=synth | _lib.FP64, ray=0, k=4) == _lib.EK
    assert angmf(flags=synth, ray=0, out=FAKE) == _lib.EALIAS
    assert angmf(flags=synth, ray=0, H=0) == _lib.OK
    assert angmf(flags=0, ray=0) == _lib.ENULL


def test_build_ray8_rejects():
    assert _lib.build_ray8_f32(FAKE, 100.0, 10.0, 100.0, 10.0, -1, 4) == _lib.ESHAPE
    assert _lib.last_error().startswith("build_ray8: ")
    assert _lib.build_ray8_f32(0, 100.0, 10.0, 100.0, 10.0, 4, 4) == _lib.ENULL
    assert _lib.build_ray8_f32(0, 100.0, 10.0, 100.0, 10.0, 0, 4) == _lib.OK


def test_empty_shapes_are_no_ops():
    # the reference returns before launching when H*W == 0 (src/dsine_ops.cu:162,179)
    assert angmf(H=0) == _lib.OK
    assert angmf(W=0, pred_norm=0) == _lib.OK
    assert angmf(B=0) == _lib.OK
    assert _lib.ray_relu_f32(0, 0, 1, 0, 5, 0) == _lib.OK


@pytest.mark.parametrize("args,code", [
    ((FAKE, FAKE + 0x10000, -1, 2, 2, 0), _lib.ESHAPE),
    ((0, FAKE, 1, 2, 2, 0), _lib.ENULL),
    ((FAKE, FAKE + 8, 1, 2, 2, 0), _lib.EALIAS),
    ((FAKE, FAKE + 0x10000, 1, 2, 2, -1), _lib.ESHAPE),
])
def test_ray_relu_rejects(args, code):
    assert _lib.ray_relu_f32(*args) == code
    assert _lib.last_error().startswith("ray_relu: ")


def upsample(**kw):
    # x 1x3x4x4 at FAKE, mask 1x576x4x4 at FAKE + 0x100000, out 1x3x32x32 beyond
    args = dict(x=FAKE, mask=FAKE + 0x100000, B=1, C=3, H=4, W=4, scale=8, normalize=True,
                eps=1e-12, out=FAKE + 0x200000, flags=0, stream=0)
    args.update(kw)
    return _lib.convex_upsample_f32(**args)


@pytest.mark.parametrize("kw,code", [
    (dict(B=-1), _lib.ESHAPE), (dict(W=-1), _lib.ESHAPE), (dict(C=0), _lib.ESHAPE),
    (dict(scale=0), _lib.ESHAPE),
    (dict(C=5), _lib.EUNSUP), (dict(scale=17), _lib.EUNSUP),
    (dict(x=0), _lib.ENULL), (dict(mask=0), _lib.ENULL), (dict(out=0), _lib.ENULL),
    (dict(flags=2), _lib.EFLAGS),
    (dict(out=FAKE + 64), _lib.EALIAS),                 # inside x
    (dict(out=FAKE + 0x100000 + 0x9000 - 16), _lib.EALIAS),  # last bytes of mask
    (dict(H=1 << 15, W=1 << 15), _lib.ESIZE),            # 2^30 pixels per sample
])
def test_upsample_rejects(kw, code):
    assert upsample(**kw) == code
    assert _lib.last_error().startswith("convex_upsample: ")


def test_upsample_empty_is_no_op():
    assert upsample(B=0) == _lib.OK
    assert upsample(H=0, x=0, mask=0, out=0) == _lib.OK
    assert upsample(W=0, normalize=False) == _lib.OK


def test_cpp_dropin_error_paths():
    assert os.path.exists(CPP_TEST), "build() compiles tests/cpp/test_dsine_ops"
    proc = subprocess.run([CPP_TEST, "cpu"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout


def test_recompute_ratio_query():
    """The cancellation threshold the fast path recomputes below, per window
    size: positive for the fp32 path (the same with the activations formed in
    the kernel), 0 for the double-precision kernel, -1 for a window size the
    op rejects."""
    for k in (1, 3, 5, 7, 9):
        t = _lib.angmf_recompute_ratio(k, _lib.DEFAULT)
        assert 0.0 < t < 1e-2
        assert _lib.angmf_recompute_ratio(k, _lib.LOGITS) == t
        assert _lib.angmf_recompute_ratio(k, _lib.FP64) == 0.0
        assert _lib.angmf_recompute_ratio(k, _lib.FP64 | _lib.LOGITS) == 0.0
    for k in (0, 2, 11, -1):
        assert _lib.angmf_recompute_ratio(k) == -1.0


def _dynsyms(path, *flags):
    return subprocess.run(["nm", "-D", "-C", *flags, path], stdout=subprocess.PIPE, text=True,
                          check=True).stdout.splitlines()


def test_c_abi_library_exports_only_the_c_abi():
    """libbvml_dsine.so adds nothing but bvml_dsine_* to a process: no
    brovisionml::dsine symbol that could collide with brovisionml's own
    src/dsine_ops.cpp, no brotensor symbol."""
    names = [ln.split()[-1] for ln in _dynsyms(LIB, "--defined-only")
             if ln.split()[1] in "TDBRVWiu"]
    extra = [n for n in names if not n.startswith("bvml_dsine_")]
    assert extra == []
    assert sorted(n for n in names) == sorted(declared_functions())


def test_cxx_layer_exports_only_the_dropin():
    from brovisionml_amd.build import LIB_CXX
    defined = [ln.split(None, 2)[2] for ln in _dynsyms(LIB_CXX, "--defined-only")
               if " T " in ln or " W " in ln]
    assert defined and all(n.startswith("brovisionml::dsine::") for n in defined)
    for fn in ("ray_relu(", "angmf_propagate(", "angmf_propagate_logits(",
               "convex_upsample(", "convex_upsample_normalize("):
        assert any(n.startswith(f"brovisionml::dsine::{fn}") for n in defined), fn
    # brotensor::Tensor comes from outside: brotensor in a brovisionml build
    undefined = [ln for ln in _dynsyms(LIB_CXX, "--undefined-only") if "brotensor::" in ln]
    assert undefined


def test_refiner_libraries_export_only_their_interfaces():
    """libbvml_dsine_refine.so adds bvml_dsine_refiner_* (the declarations of
    include/bvml_dsine_refine.h) and nothing else; libbvml_dsine_refine_cxx.so
    adds brovisionml::dsine::Refiner's members and nothing else, so a
    brovisionml build can take the ops' C++ layer and the Refiner class
    independently, each in place of exactly one of its own sources."""
    import re
    from brovisionml_amd.build import LIB_CXX, LIB_REFINE, LIB_REFINE_CXX, INCLUDE
    names = [ln.split()[-1] for ln in _dynsyms(LIB_REFINE, "--defined-only")
             if ln.split()[1] in "TDBRVWiu"]
    with open(os.path.join(INCLUDE, "bvml_dsine_refine.h")) as f:
        declared = set(re.findall(r"\b(bvml_dsine_refiner_\w+)\s*\(", f.read()))
    assert sorted(names) == sorted(declared)
    defined = [ln.split(None, 2)[2] for ln in _dynsyms(LIB_REFINE_CXX, "--defined-only")
               if " T " in ln or " W " in ln]
    assert defined and all(n.startswith("brovisionml::dsine::Refiner::") for n in defined)
    for fn in ("load(", "load_file(", "to(", "device(", "forward(", "Refiner()"):
        assert any(n.startswith(f"brovisionml::dsine::Refiner::{fn}") for n in defined), fn
    ops = {ln.split(None, 2)[2] for ln in _dynsyms(LIB_CXX, "--defined-only")
           if " T " in ln or " W " in ln}
    assert not ops & set(defined)


def test_cxx_layer_compiles_against_brotensors_api():
    """dsine_ops.cpp and the launchers header use only the brotensor::Tensor
    members and Device enumerators brovisionml's own sources use."""
    from brovisionml_amd import build
    build.check_brotensor_api()


def _intr(H, W):
    from brovisionml_amd import workloads as wl
    return wl.scaled_intrinsics(wl.intrins_from_fov(8 * H, 8 * W, 60.0), H, W, 8 * H, 8 * W)


def test_plan_of_the_workloads():
    """The launch plan per workload (host logic only): run-split kernels on
    the small images (8 waves per group where 4 would leave CUs idle; range
    tiles, reported as tile_h 0, where W = 80 is not a whole number of
    64-pixel groups), the whole-window kernel on 4 x 512 x 512 at k = 7."""
    from brovisionml_amd import workloads as wl
    want = {0: (True, 8, 64, 0), 1: (True, 8, 64, 1), 2: (True, 4, 64, 2), 3: (True, 2, 256, 0),
            4: (True, 1, 64, 8)}
    for w in wl.WORKLOADS:
        _, intr = w.intrinsics()
        assert _lib.angmf_plan(w.B, w.H, w.W, w.k, *intr) == want[w.index], w.name
    # FP64 flag, and intrinsics outside the fast path's range: the fp64 kernel
    assert _lib.angmf_plan(1, 64, 64, 5, *_intr(64, 64), flags=_lib.FP64)[0] is False
    assert _lib.angmf_plan(1, 64, 64, 5, 1e-4, 32.0, 1e-4, 32.0)[0] is False
    with pytest.raises(RuntimeError, match="k must be"):
        _lib.angmf_plan(1, 4, 4, 4, 1.0, 2.0, 1.0, 2.0)
    with pytest.raises(RuntimeError, match="flag"):
        _lib.angmf_plan(1, 4, 4, 5, 1.0, 2.0, 1.0, 2.0, flags=64)


def test_plan_layout_rules():
    """The layout choice (host logic only): the whole-window kernel once a
    launch fills the resident whole-window workgroups (512: two per CU) and
    its last round at least 60% of the way; more waves per group when the
    first choice leaves CUs idle (fewer than 256 workgroups); at k = 9 a
    64-wide tile's halo needs the 8 waves' threads to stage it."""
    cases = {(1, 512, 512, 5): 1, (4, 256, 256, 5): 1, (1, 1030, 512, 5): 1,
             (1, 512, 512, 7): 1, (2, 384, 384, 5): 4, (3, 256, 256, 5): 4,
             (1, 256, 256, 5): 4, (1, 96, 96, 5): 8, (1, 200, 200, 5): 4,
             (1, 128, 128, 3): 4, (1, 256, 256, 3): 2, (1, 512, 512, 9): 8}
    for (B, H, W, k), g in cases.items():
        assert _lib.angmf_plan(B, H, W, k, *_intr(H, W))[1] == g, (B, H, W, k)
    # non-temporal plane loads: whole-window launches past the 256 MB cache
    assert _lib.angmf_plan_full(4, 512, 512, 7, *_intr(512, 512))[4] is True
    assert _lib.angmf_plan_full(1, 800, 800, 5, *_intr(800, 800))[4] is True
    assert _lib.angmf_plan_full(2, 512, 512, 5, *_intr(512, 512))[4] is False
    assert _lib.angmf_plan_full(1, 256, 256, 5, *_intr(256, 256))[4] is False


# Every (k, waves per group) the fp32 kernel is instantiated for
# (kGChoices, kGSmall and kWholeWindowOk in brovisionml_amd/csrc/dsine_ops.hip).
KERNEL_LAYOUTS = {(1, 1), (3, 2), (3, 4), (5, 1), (5, 2), (5, 4), (5, 8), (7, 1), (7, 4), (7, 8),
                  (9, 8)}


def test_gpu_parity_shapes_cover_every_kernel_layout():
    """The GPU parity shapes reach every instantiated (k, waves per group)
    layout of the fp32 kernel (1: whole window; 2, 4, 8: runs) and its
    whole-window variant with logits and rays from the intrinsics."""
    from tests.test_gpu_parity import SHAPES
    got = {(k, _lib.angmf_plan(B, H, W, k, *_intr(H, W))[1]) for B, H, W, k in SHAPES}
    assert got == KERNEL_LAYOUTS, (KERNEL_LAYOUTS - got, got - KERNEL_LAYOUTS)
    # the whole-window kernels with and without non-temporal plane loads
    whole = {(k, _lib.angmf_plan_full(B, H, W, k, *_intr(H, W))[4]) for B, H, W, k in SHAPES
             if k in (5, 7) and _lib.angmf_plan(B, H, W, k, *_intr(H, W))[1] == 1}
    assert whole == {(5, False), (5, True), (7, True)}, whole
    flags = _lib.LOGITS | _lib.RAY_FROM_INTRINSICS
    assert _lib.angmf_plan(2, 512, 512, 5, *_intr(512, 512), flags=flags)[1] == 1
