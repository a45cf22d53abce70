"""Host side of the native refiner (libbvml_dsine_refine.so,
include/bvml_dsine_refine.h), no GPU: its exports, the checkpoint tensors it
reads, its safetensors reader (F32, F16 and BF16 widened to fp32 as the
reference's loader widens them, src/weights_util.h:27-63; the missing-tensor
and size errors of src/dsine_refine.cpp:32-66), the argument checks that
forward makes before any HIP call, and the host path of the loop
(bvml_dsine_refiner_forward_cpu) against the CPU restatement
(oracle/refiner.py) and the closed-form pins of tests/refiner_pins.py."""
from __future__ import annotations

import ctypes
import json
import os
import struct

import numpy as np
import pytest

from brovisionml_amd import _lib, refiner as rf

FAKE = 1 << 20  # a non-NULL address that is never dereferenced


@pytest.fixture(scope="module")
def lib():
    return _lib.load_refine()


def test_exports(lib):
    for name in _lib.REFINE_EXPORTS:
        assert hasattr(lib, name), name


def test_tensor_numel(lib):
    for name, shape in rf.weight_shapes().items():
        assert lib.bvml_dsine_refiner_tensor_numel(name.encode()) == int(np.prod(shape)), name
    for bad in (b"gru.convz", b"decoder.x.weight", b"", b"prob_head.1.weight"):
        assert lib.bvml_dsine_refiner_tensor_numel(bad) == -1
    assert lib.bvml_dsine_refiner_tensor_numel(None) == -1


def test_set_get_roundtrip():
    w = rf.random_weights(4)
    r = rf.NativeRefiner(w)
    for k, v in w.items():
        assert np.array_equal(r.get_tensor(k).view(np.uint32), v.reshape(-1).view(np.uint32)), k


def test_set_tensor_errors(lib):
    r = rf.NativeRefiner()
    a = np.zeros(64, np.float32)
    assert lib.bvml_dsine_refiner_set_tensor(r._h, b"gru.convz.bias", a.ctypes.data, 63) == \
        _lib.EWEIGHTS
    assert "64" in _lib.refine_last_error()
    assert lib.bvml_dsine_refiner_set_tensor(r._h, b"nope", a.ctypes.data, 64) == _lib.EWEIGHTS
    assert "unknown tensor 'nope'" in _lib.refine_last_error()
    assert lib.bvml_dsine_refiner_set_tensor(r._h, b"gru.convz.bias", None, 64) == _lib.ENULL
    with pytest.raises(RuntimeError, match="not set"):
        r.get_tensor("gru.convz.bias")


# ---- safetensors files written byte by byte
def _dtype_bytes(v: np.ndarray, dtype: str) -> bytes:
    if dtype == "F32":
        return np.ascontiguousarray(v, "<f4").tobytes()
    if dtype == "F16":
        return np.ascontiguousarray(v.astype("<f2")).tobytes()
    if dtype == "BF16":
        bits = np.ascontiguousarray(v, "<f4").view("<u4") >> 16  # truncation: exact for
        return bits.astype("<u2").tobytes()                      # bf16-representable values
    if dtype == "I32":
        return np.ascontiguousarray(v.astype("<i4")).tobytes()
    raise ValueError(dtype)


def write_safetensors(path, tensors: dict, dtypes: dict | None = None, shapes: dict | None = None,
                      metadata: dict | None = None, header_patch=None, truncate: int = 0):
    """tensors: name -> float32 array; dtypes/shapes override per name."""
    dtypes, shapes = dtypes or {}, shapes or {}
    header, blobs, at = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, v in tensors.items():
        dt = dtypes.get(name, "F32")
        b = _dtype_bytes(v, dt)
        header[name] = {"dtype": dt, "shape": list(shapes.get(name, v.shape)),
                        "data_offsets": [at, at + len(b)]}
        blobs.append(b)
        at += len(b)
    if header_patch:
        header_patch(header)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    data = struct.pack("<Q", len(h)) + h + b"".join(blobs)
    if truncate:
        data = data[:-truncate]
    with open(path, "wb") as f:
        f.write(data)


def _bf16_exact(w: dict) -> dict:
    return {k: (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32) for k, v in w.items()}


@pytest.mark.parametrize("dtype", ["F32", "F16", "BF16"])
def test_load_file_dtypes(tmp_path, dtype):
    w = rf.random_weights(9)
    if dtype == "BF16":
        w = _bf16_exact(w)
    # F16 covers normals, subnormals, zero and infinities
    if dtype == "F16":
        w["gru.convz.bias"][:8] = [0.0, -0.0, 6e-8, -3e-6, 65504.0, np.inf, -np.inf, 1e-5]
    path = str(tmp_path / "model.safetensors")
    extra = {"decoder.conv.weight": np.ones((3, 3), np.float32)}
    write_safetensors(path, {**extra, **w}, dtypes={k: dtype for k in w},
                      metadata={"format": "pt", "note": "esc \"\\u00e9\" \u00e9 \ud83d\ude00"})
    r = rf.NativeRefiner(path=path)
    for k, v in w.items():
        want = v.astype(np.float16).astype(np.float32) if dtype == "F16" else v
        got = r.get_tensor(k)
        assert np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32)), k


def test_load_file_matches_safetensors_library(tmp_path):
    """A file written by the safetensors package itself."""
    from safetensors.numpy import save_file
    w = rf.random_weights(10)
    path = str(tmp_path / "lib.safetensors")
    save_file(w, path, metadata={"format": "np"})
    r = rf.NativeRefiner(path=path)
    for k, v in w.items():
        assert np.array_equal(r.get_tensor(k), v.reshape(-1)), k


def _expect_load_error(tmp_path, status, match, **kw):
    w = rf.random_weights(12)
    good = rf.random_weights(13)
    path = str(tmp_path / "bad.safetensors")
    tensors = kw.pop("tensors", w)
    write_safetensors(path, tensors, **kw)
    r = rf.NativeRefiner(good)
    st = r._lib.bvml_dsine_refiner_load_file(r._h, path.encode())
    assert st == status, (st, _lib.refine_last_error())
    assert match in _lib.refine_last_error()
    # nothing changed
    for k, v in good.items():
        assert np.array_equal(r.get_tensor(k), v.reshape(-1)), k


def test_load_file_errors(tmp_path):
    w = rf.random_weights(12)
    missing = {k: v for k, v in w.items() if k != "xy_head.2.bias"}
    _expect_load_error(tmp_path, _lib.EWEIGHTS, "missing tensor 'xy_head.2.bias'", tensors=missing)
    _expect_load_error(tmp_path, _lib.EWEIGHTS, "unsupported dtype I32",
                       dtypes={"gru.convq.bias": "I32"})
    wrong = dict(w)
    wrong["prob_head.4.weight"] = np.zeros((24, 64, 1, 1), np.float32)
    _expect_load_error(tmp_path, _lib.EWEIGHTS, "'prob_head.4.weight' has 1536 elements, expected "
                       "1600", tensors=wrong)
    _expect_load_error(tmp_path, _lib.EWEIGHTS, "output channels",
                       shapes={"gru.convz.bias": (1, 64)})

    def bad_offsets(h):
        h["gru.convr.bias"]["data_offsets"][1] += 4
    _expect_load_error(tmp_path, _lib.EFILE, "bad data offsets", header_patch=bad_offsets)

    def negative_offsets(h):
        h["gru.convr.bias"]["data_offsets"][0] = -4
    _expect_load_error(tmp_path, _lib.EFILE, "malformed entry", header_patch=negative_offsets)
    _expect_load_error(tmp_path, _lib.EFILE, "bad data offsets", truncate=4)


def test_load_file_bad_files(tmp_path, lib):
    r = rf.NativeRefiner()
    p = str(tmp_path / "x.safetensors")
    cases = [
        (b"", "too short"),
        (struct.pack("<Q", 0), "bad header length"),
        (struct.pack("<Q", 1 << 40) + b"{}", "bad header length"),
        (struct.pack("<Q", 5) + b"{oops", "malformed JSON"),
        (struct.pack("<Q", 2) + b"[]", "malformed JSON"),
        (struct.pack("<Q", 4) + b'{"a"', "malformed JSON"),
        (struct.pack("<Q", 2) + b"{}", "missing tensor 'gru.convz.weight'"),
    ]
    for data, match in cases:
        with open(p, "wb") as f:
            f.write(data)
        st = lib.bvml_dsine_refiner_load_file(r._h, p.encode())
        assert st in (_lib.EFILE, _lib.EWEIGHTS), (data, st)
        assert match in _lib.refine_last_error(), (data, _lib.refine_last_error())
    st = lib.bvml_dsine_refiner_load_file(r._h, str(tmp_path / "absent").encode())
    assert st == _lib.EFILE and "cannot open" in _lib.refine_last_error()
    assert lib.bvml_dsine_refiner_load_file(r._h, None) == _lib.ENULL


# ---- forward's checks (all before its first HIP call)
def _forward(lib, r, **kw):
    a = dict(normal=FAKE, feature=FAKE + (1 << 24), hidden=FAKE + (1 << 26), h8=8, w8=8,
             fx=64.0, fy=64.0, cx=32.0, cy=32.0, orig_h=64, orig_w=64, pad_t=0, pad_l=0,
             out_h=64, out_w=64, out=FAKE + (1 << 28), coarse=None, stream=None)
    a.update(kw)
    return lib.bvml_dsine_refiner_forward(r, a["normal"], a["feature"], a["hidden"], a["h8"],
                                          a["w8"], a["fx"], a["fy"], a["cx"], a["cy"],
                                          a["orig_h"], a["orig_w"], a["pad_t"], a["pad_l"],
                                          a["out_h"], a["out_w"], a["out"], a["coarse"],
                                          a["stream"])


def test_forward_checks(lib):
    empty = rf.NativeRefiner()
    full = rf.NativeRefiner(rf.random_weights(1))
    assert _forward(lib, None) == _lib.ENULL
    assert _forward(lib, full._h, out=None) == _lib.ENULL
    assert _forward(lib, full._h, h8=0) == _lib.ESHAPE
    assert _forward(lib, full._h, orig_w=0) == _lib.ESHAPE
    assert _forward(lib, full._h, pad_t=1) == _lib.ESHAPE         # 1 + 64 rows > 64
    assert "must lie inside the 64 x 64 result" in _lib.refine_last_error()
    assert _forward(lib, full._h, pad_l=-1, out_w=10) == _lib.ESHAPE
    assert _forward(lib, full._h, out_h=0) == _lib.ESHAPE
    assert _forward(lib, full._h, h8=1 << 14, w8=1 << 14, orig_h=1 << 17, orig_w=1 << 17) == \
        _lib.ESIZE
    assert _forward(lib, full._h, fx=0.0) == _lib.EPARAM
    assert _forward(lib, full._h, cy=float("nan")) == _lib.EPARAM
    assert _forward(lib, empty._h) == _lib.EWEIGHTS
    assert "tensor 'gru.convz.weight' not set" in _lib.refine_last_error()
    assert _forward(lib, full._h, out=FAKE + 16) == _lib.EALIAS
    assert _forward(lib, full._h, coarse=FAKE + (1 << 26) + 64) == _lib.EALIAS
    assert _forward(lib, full._h, coarse=FAKE + (1 << 28) + 4) == _lib.EALIAS


def test_destroy_null(lib):
    lib.bvml_dsine_refiner_destroy(None)
    assert lib.bvml_dsine_refiner_create(None) == _lib.ENULL
    h = ctypes.c_void_p()
    assert lib.bvml_dsine_refiner_create(ctypes.byref(h)) == _lib.OK
    lib.bvml_dsine_refiner_destroy(h)
    assert os.path.exists(_lib.LIB_REFINE)


# ---- the host path (bvml_dsine_refiner_forward_cpu) against the restatement and the pins
def _cpu_dec(arrays):
    import torch
    return rf.DecoderOutput(*(torch.from_numpy(np.ascontiguousarray(a))[None] for a in arrays))


@pytest.mark.parametrize("H,W,fov,seed", [(12, 16, 60.0, 3), (9, 7, 90.0, 4)])
def test_cpu_forward_matches_oracle(H, W, fov, seed):
    """fp32 convolutions against the restatement's float64 ones through five
    iterations: 1e-4 per component, the device path's bar."""
    from oracle import refiner as oref
    from brovisionml_amd import workloads as wl
    from tests import refiner_pins as pins
    weights = rf.random_weights(seed)
    n, feature, hidden = pins.inputs(H, W, seed)
    intr = wl.intrins_from_fov(8 * H, 8 * W, fov)
    fuv = wl.scaled_intrinsics(intr, H, W, 8 * H, 8 * W)
    out, coarse = rf.NativeRefiner(weights).forward(_cpu_dec((n, feature, hidden)), intr,
                                                    8 * H, 8 * W, coarse=True)
    want = []
    oref.refine_forward(weights, n, feature, hidden, intr, fuv,
                        wl.build_ray8(intr, H, W, 8 * H, 8 * W).reshape(3, H, W),
                        rf.uv_map(intr, H, W, 8 * H, 8 * W), trace=want, nthreads=8)
    for it, (wp, _) in enumerate(want):
        assert np.abs(coarse[it].numpy().astype(np.float64) - wp).max() <= 1e-4, it
    assert np.abs(out[0].numpy().astype(np.float64) - want[-1][1]).max() <= 1e-4


def test_cpu_forward_pins_and_crop():
    """The closed-form pins (constant heads: each iteration one direct
    propagate; a one-hot up mask: the clamped tap), the crop as a slice of
    the whole map, and a result that does not depend on the thread count."""
    from tests import refiner_pins as pins
    H, W = 12, 16
    n, feature, hidden, intr, fuv, ray8, _ = pins.setup(H, W, 60.0, 7)
    dec = _cpu_dec((n, feature, hidden))
    w, data = pins.pinned_weights("const_heads", 7)
    _, coarse = rf.NativeRefiner(w).forward(dec, intr, 8 * H, 8 * W, coarse=True)
    chain = list(coarse.numpy())
    for p, wp in zip(chain, pins.const_heads_expected(data, n, ray8, fuv, H, W, chain=chain)):
        assert np.abs(p.astype(np.float64) - wp).max() <= 1e-5
    w, _ = pins.pinned_weights("onehot_up", 7, n0=5)
    model = rf.NativeRefiner(w)
    out, coarse = model.forward(dec, intr, 8 * H, 8 * W, coarse=True)
    assert np.abs(out[0].numpy() - pins.onehot_up_expected(coarse[-1].numpy(), 5)).max() <= 1e-5
    crop = rf.Crop(orig_h=8 * H - 11, orig_w=8 * W - 6, pad_t=5, pad_l=3)
    part = model.forward(dec, intr, 8 * H, 8 * W, crop=crop, nthreads=1)
    assert part.shape == (1, 3, crop.orig_h, crop.orig_w)
    assert np.array_equal(part.numpy(), out.numpy()[:, :, 5:5 + crop.orig_h, 3:3 + crop.orig_w])


# ---- the C++ class (tests/cpp/test_dsine_refine.cpp over libbvml_dsine_cxx.so)
CPP_REFINE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build",
                          "test_dsine_refine")


def write_case(path, n, feature, hidden, intr, orig_h, orig_w, crop):
    """The case file tests/cpp/test_dsine_refine.cpp reads."""
    H, W = n.shape[1:]
    with open(path, "wb") as f:
        f.write(struct.pack("<8i", H, W, orig_h, orig_w, crop.pad_t, crop.pad_l, crop.orig_h,
                            crop.orig_w))
        f.write(struct.pack("<4f", intr.fx, intr.fy, intr.cx, intr.cy))
        for a in (n, feature, hidden):
            f.write(np.ascontiguousarray(a, "<f4").tobytes())


def cpp_case(tmp_path, seed=21, H=10, W=13):
    """(weights file, case file, weights, maps, intrinsics, crop) for a run."""
    from safetensors.numpy import save_file
    from brovisionml_amd import workloads as wl
    from tests import refiner_pins as pins
    weights = rf.random_weights(seed)
    wpath = str(tmp_path / "model.safetensors")
    save_file(weights, wpath)
    maps = pins.inputs(H, W, seed)
    intr = wl.intrins_from_fov(8 * H, 8 * W, 65.0)
    crop = rf.Crop(orig_h=8 * H - 9, orig_w=8 * W - 4, pad_t=4, pad_l=2)
    cpath = str(tmp_path / "case.bin")
    write_case(cpath, *maps, intr, 8 * H, 8 * W, crop)
    return wpath, cpath, weights, maps, intr, crop


def run_cpp_refine(*args, timeout=300):
    import subprocess
    assert os.path.exists(CPP_REFINE), "build() compiles tests/cpp/test_dsine_refine"
    proc = subprocess.run([CPP_REFINE, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=timeout)
    return proc.returncode, proc.stdout


def test_cpp_refiner_errors():
    rc, out = run_cpp_refine("errors")
    assert rc == 0 and "OK" in out, out


def test_cpp_refiner_cpu(tmp_path):
    """Refiner::load_file, to(CPU), forward with a crop: the native refiner's
    host path, bit for bit."""
    wpath, cpath, weights, maps, intr, crop = cpp_case(tmp_path)
    opath = str(tmp_path / "out.bin")
    rc, out = run_cpp_refine("run", "cpu", wpath, cpath, opath)
    assert rc == 0 and "OK" in out, out
    got = np.fromfile(opath, np.float32).reshape(1, 3, crop.orig_h, crop.orig_w)
    H, W = maps[0].shape[1:]
    want = rf.NativeRefiner(weights).forward(_cpu_dec(maps), intr, 8 * H, 8 * W, crop=crop)
    assert np.array_equal(got.view(np.uint32), want.numpy().view(np.uint32))
