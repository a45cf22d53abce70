"""CPU parity oracle -- TEST INFRASTRUCTURE ONLY.

ctypes binding of oracle/_build/liboracle_dsine.so, the double-precision C
restatement of brovisionml's CPU twin (src/dsine_ops.cpp:24-172) and of the
refiner's convex upsample + L2 normalise (src/dsine_refine.cpp:276-282,
spec include/brovisionml/dsine_refine.h:91-97).  Only the
tests, the smoke check and the CPU-baseline leg of the benchmark may use it,
to check results or as the timed CPU reference; the product never does.

`Oracle(path)` binds any build of oracle/dsine_ops_oracle.c (the mutation
test loads deliberately broken ones); the module-level functions use the
default build.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle_dsine.so")
SOURCE = os.path.join(HERE, "dsine_ops_oracle.c")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def compile_variant(out_path: str, mutation: int = 0) -> str:
    """Build the oracle with ORACLE_MUTATION=mutation into out_path (gcc, the
    flags of oracle/Makefile)."""
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
                    "-fopenmp", "-shared", f"-DORACLE_MUTATION={mutation}", "-o", out_path,
                    SOURCE, "-lm"], check=True)
    return out_path


class Oracle:
    def __init__(self, path: str = LIB):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library {path} missing; run `make -C oracle`")
        lib = ctypes.CDLL(path)
        vp, i, ll, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_double
        lib.oracle_axis_angle_to_matrix.argtypes = [d, d, d, vp]
        lib.oracle_axis_angle_to_matrix.restype = None
        lib.oracle_axis.argtypes = [d] * 11 + [vp]
        lib.oracle_axis.restype = None
        lib.oracle_ray_relu_vec.argtypes = [d] * 6 + [vp]
        lib.oracle_ray_relu_vec.restype = None
        lib.oracle_neighbour.argtypes = [d] * 15 + [vp]
        lib.oracle_neighbour.restype = None
        lib.oracle_ray_relu_f32.argtypes = [vp, vp, i, i, i, ll]
        lib.oracle_ray_relu_f32.restype = None
        lib.oracle_angmf_propagate_rows_f32.argtypes = [
            vp, vp, vp, vp, vp, d, d, d, d, i, i, i, i, ll, vp, vp, vp, i, i, i]
        lib.oracle_angmf_propagate_rows_f32.restype = None
        lib.oracle_convex_upsample_f32.argtypes = [
            vp, vp, i, i, i, i, i, i, d, vp, i]
        lib.oracle_convex_upsample_f32.restype = None
        self.lib = lib

    def axis_angle_to_matrix(self, v) -> np.ndarray:
        R = np.zeros(9, dtype=np.float64)
        self.lib.oracle_axis_angle_to_matrix(float(v[0]), float(v[1]), float(v[2]), _ptr(R))
        return R.reshape(3, 3)

    def axis(self, n, pix, xy, intr) -> np.ndarray:
        a = np.zeros(3, dtype=np.float64)
        fu, cu, fv, cv = intr
        self.lib.oracle_axis(float(n[0]), float(n[1]), float(n[2]), float(pix[0]),
                             float(pix[1]), float(xy[0]), float(xy[1]), fu, cu, fv, cv, _ptr(a))
        return a

    def ray_relu_vec(self, n, r) -> np.ndarray:
        o = np.zeros(3, dtype=np.float64)
        self.lib.oracle_ray_relu_vec(*(float(v) for v in n), *(float(v) for v in r), _ptr(o))
        return o

    def neighbour(self, n, pix, xy, theta, r, intr) -> np.ndarray:
        o = np.zeros(3, dtype=np.float64)
        fu, cu, fv, cv = intr
        self.lib.oracle_neighbour(float(n[0]), float(n[1]), float(n[2]), float(pix[0]),
                                  float(pix[1]), float(xy[0]), float(xy[1]), float(theta),
                                  float(r[0]), float(r[1]), float(r[2]), fu, cu, fv, cv, _ptr(o))
        return o

    def ray_relu(self, normal, ray, H: int, W: int) -> np.ndarray:
        """RayReLU(normal) as a new float32 array of normal's shape.
        ray: 3*H*W (shared) or B*3*H*W (per sample)."""
        n = _f32c(normal).copy()
        r = _f32c(ray)
        HW = H * W
        B = n.size // (3 * HW) if HW else 0
        bstride = 0 if r.size == 3 * HW else 3 * HW
        self.lib.oracle_ray_relu_f32(_ptr(n), _ptr(r), B, H, W, bstride)
        return n

    def angmf_propagate(self, pred_norm, prob, xy, angle, ray, intr, H: int, W: int,
                        k: int = 5, rows=None, nthreads: int = 1, return_acc: bool = False,
                        return_qs: bool = False):
        """angmf_propagate over all B samples (inferred from pred_norm).
        rows=(y0, y1) limits the output rows computed (others stay NaN).
        Returns out (float32, pred_norm's shape) [and the double accumulator
        (pred_norm's shape)] [and sum over neighbours of (prob/|p|)^2, shaped
        (B, H*W)], p a neighbour's RayReLU'd vector before its normalise."""
        pn, pr, xyp, ap, rp = (_f32c(a) for a in (pred_norm, prob, xy, angle, ray))
        HW = H * W
        B = pn.size // (3 * HW)
        bstride = 0 if rp.size == 3 * HW else 3 * HW
        out = np.full(pn.shape, np.nan, dtype=np.float32)
        acc = np.full(pn.shape, np.nan, dtype=np.float64) if return_acc else None
        qs = np.full((B, HW), np.nan, dtype=np.float64) if return_qs else None
        y0, y1 = rows if rows is not None else (0, H)
        fu, cu, fv, cv = intr
        self.lib.oracle_angmf_propagate_rows_f32(
            _ptr(pn), _ptr(pr), _ptr(xyp), _ptr(ap), _ptr(rp), fu, cu, fv, cv, B, H, W, k,
            bstride, _ptr(out), _ptr(acc) if acc is not None else None,
            _ptr(qs) if qs is not None else None, y0, y1, nthreads)
        res = (out,) + ((acc,) if return_acc else ()) + ((qs,) if return_qs else ())
        return res if len(res) > 1 else out


    def convex_upsample(self, x, mask, H: int, W: int, s: int = 8, normalize: bool = True,
                        eps: float = 1e-12, nthreads: int = 1) -> np.ndarray:
        """Convex upsample by s (9-tap softmax mask, replicate padding), then
        the channel L2-normalise when `normalize`.  x: (B, C, H*W) or
        (B, C, H, W); mask: (B, 9*s*s, ...).  Returns (B, C, s*H, s*W) float32."""
        xf, mf = _f32c(x), _f32c(mask)
        HW = H * W
        B = mf.size // (9 * s * s * HW)
        C = xf.size // (B * HW)
        if C > 16:
            raise ValueError("oracle convex_upsample: at most 16 channels")
        out = np.full((B, C, s * H, s * W), np.nan, dtype=np.float32)
        self.lib.oracle_convex_upsample_f32(_ptr(xf), _ptr(mf), B, C, H, W, s,
                                            1 if normalize else 0, float(eps), _ptr(out), nthreads)
        return out


_default = None


def default() -> Oracle:
    global _default
    if _default is None:
        _default = Oracle(LIB)
    return _default


def load():
    return default().lib


def axis_angle_to_matrix(v):
    return default().axis_angle_to_matrix(v)


def axis(n, pix, xy, intr):
    return default().axis(n, pix, xy, intr)


def ray_relu_vec(n, r):
    return default().ray_relu_vec(n, r)


def neighbour(n, pix, xy, theta, r, intr):
    return default().neighbour(n, pix, xy, theta, r, intr)


def ray_relu(normal, ray, H, W):
    return default().ray_relu(normal, ray, H, W)


def angmf_propagate(*args, **kwargs):
    return default().angmf_propagate(*args, **kwargs)


def convex_upsample(*args, **kwargs):
    return default().convex_upsample(*args, **kwargs)
