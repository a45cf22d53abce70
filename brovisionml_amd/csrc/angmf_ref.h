// The DSINE ops' per-pixel arithmetic in double precision and in the
// reference's own operation order, for the host and the device alike: the
// CPU branch of the public dispatch (dsine_ops_cpu.cpp) runs it for CPU
// tensors, and the GPU kernels (dsine_ops.hip) run it as their
// reference-order tier and as the BVML_DSINE_FP64 kernel.  With contraction
// off and IEEE division and square root, the host build reproduces
// brovisionml's CPU twin (src/dsine_ops.cpp:55-172) bit for bit.
#pragma once

#include <cmath>

// Host and device under hipcc; host only under a plain C++ compiler, which is
// how the CPU branch also builds.
#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define BVML_HD __host__ __device__
#else
#define BVML_HD
#endif

// No fused multiply-adds in the functions below: clang takes the pragma;
// g++ builds of the CPU branch pass -ffp-contract=off.
#if defined(__clang__)
#define BVML_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define BVML_NO_CONTRACT
#endif

namespace bvml {

using std::cos;
using std::exp;
using std::fabs;
using std::isfinite;
using std::sin;
using std::sqrt;

struct Ray3f {
    float x, y, z;
};

// src/dsine_ops.cpp:27: the float 1e-2f, widened to double where the
// reference does arithmetic in double.
constexpr float kRayEpsF = 1e-2f;

// The float pi the refiner scales the angle head by (src/dsine_refine.cpp:26).
constexpr float kPiF = 3.14159265358979323846f;

// std::max(a, b) == (a < b) ? b : a -- returns a when a is NaN, as the
// reference CPU path does (fmax would not).
BVML_HD inline double smax(double a, double b) { return (a < b) ? b : a; }

// The activations the refiner applies to the prob and angle heads
// (src/dsine_refine.cpp:262-267), as correctly rounded floats: sigmoid in
// double, rounded once; the angle's product with the float pi in float.
BVML_HD inline float sigmoid_ref(float x) {
    return (float)(1.0 / (1.0 + exp(-(double)x)));
}
BVML_HD inline float angle_ref(float x) { return sigmoid_ref(x) * kPiF; }

// The ray of pixel (x, y) as build_ray8 forms it from the grid-scaled
// intrinsics (src/dsine_decoder.cpp:252-253 and :285-290): ray_x, ray_y in
// double rounded to float, then [ray_x, ray_y, 1] normalised in double and
// each channel rounded to float.  IEEE double division and square root, in
// the host's operation order with contraction off, give the host's bits.
BVML_HD inline Ray3f synth_ray(int x, int y, double fu, double cu, double fv,
                                            double cv) {
BVML_NO_CONTRACT
    const double rx = (float)(((x + 0.5) - cu) / fu);
    const double ry = (float)(((y + 0.5) - cv) / fv);
    const double rz = 1.0;
    const double inv = 1.0 / smax(sqrt(rx * rx + ry * ry + rz * rz), 1e-12);
    return Ray3f{(float)(rx * inv), (float)(ry * inv), (float)(rz * inv)};
}

// RayReLU of one normal against one ray, src/dsine_ops.cpp:55-76 (and the
// fused copy at :150-160): c = n.r / max(|n||r|, 1e-8), then
// normalize(n + r (max(c - eps, 0) + eps - c)) with 1e-12.  pinv is the last
// normalise's 1/max(|n + diff|, 1e-12).
BVML_HD inline void ray_relu_ref(double nx, double ny, double nz, double rx,
                                             double ry, double rz, double& ox, double& oy,
                                             double& oz, double& pinv) {
BVML_NO_CONTRACT
    const double nn = sqrt(nx * nx + ny * ny + nz * nz);
    const double rr = sqrt(rx * rx + ry * ry + rz * rz);
    const double denom = smax(nn * rr, 1e-8);
    const double cs = (nx * rx + ny * ry + nz * rz) / denom;
    const double relu_cm = smax(cs - (double)kRayEpsF, 0.0) + (double)kRayEpsF;
    const double dcoef = relu_cm - cs;
    const double mx = nx + rx * dcoef, my = ny + ry * dcoef, mz = nz + rz * dcoef;
    const double inv = 1.0 / smax(sqrt(mx * mx + my * my + mz * mz), 1e-12);
    ox = mx * inv;
    oy = my * inv;
    oz = mz * inv;
    pinv = inv;
}

// One neighbour's RayReLU'd rotated normal, in the operation order of
// src/dsine_ops.cpp:110-160 (axis :110-138, axis_angle_to_matrix :31-51,
// rotate + renormalise :140-148, RayReLU :150-160).  Contraction is off so
// the sign-deciding dd is bit-identical to the CPU's.  pinv is the last
// normalise's 1/max(|p|, 1e-12).
BVML_HD inline void nbr_ref_f64(double nx, double ny, double nz, double pix_x,
                                            double pix_y, double xs, double ys, double theta,
                                            double rx, double ry, double rz, double fu,
                                            double cu, double fv, double cv, double& ox,
                                            double& oy, double& oz, double& pinv) {
BVML_NO_CONTRACT
    const double xyinv = 1.0 / smax(sqrt(xs * xs + ys * ys), 1e-12);
    xs *= xyinv;
    ys *= xyinv;
    const double du = xs / fu;
    const double dv = ys / fv;
    const double tu = (pix_x + xs - cu) / fu;
    const double tv = (pix_y + ys - cv) / fv;
    const double num = -(du * nx + dv * ny);
    double dd = tu * nx + tv * ny + nz;
    if (fabs(dd) < 1e-8) {
        const double sgn = (dd > 0.0) ? 1.0 : (dd < 0.0 ? -1.0 : 0.0);
        dd = 1e-8 * sgn;
    }
    const double dz = num / dd;
    double axx = du + dz * tu;
    double axy = dv + dz * tv;
    double axz = dz;
    const double an = sqrt(axx * axx + axy * axy + axz * axz);
    const double ainv = 1.0 / smax(an, 1e-12);
    axx *= ainv;
    axy *= ainv;
    axz *= ainv;
    if (!isfinite(axx) || !isfinite(axy) || !isfinite(axz)) axx = axy = axz = 0.0;

    // axis_angle_to_matrix(axis * theta), quaternion form.
    const double vx = axx * theta, vy = axy * theta, vz = axz * theta;
    const double angle = sqrt(vx * vx + vy * vy + vz * vz);
    const double half = angle * 0.5;
    double s;
    if (angle < 1e-6)
        s = 0.5 - (angle * angle) / 48.0;
    else
        s = sin(half) / angle;
    const double qr = cos(half);
    const double qi = vx * s, qj = vy * s, qk = vz * s;
    const double two_s = 2.0 / (qr * qr + qi * qi + qj * qj + qk * qk);
    const double R0 = 1.0 - two_s * (qj * qj + qk * qk);
    const double R1 = two_s * (qi * qj - qk * qr);
    const double R2 = two_s * (qi * qk + qj * qr);
    const double R3 = two_s * (qi * qj + qk * qr);
    const double R4 = 1.0 - two_s * (qi * qi + qk * qk);
    const double R5 = two_s * (qj * qk - qi * qr);
    const double R6 = two_s * (qi * qk - qj * qr);
    const double R7 = two_s * (qj * qk + qi * qr);
    const double R8 = 1.0 - two_s * (qi * qi + qj * qj);

    double rnx = R0 * nx + R1 * ny + R2 * nz;
    double rny = R3 * nx + R4 * ny + R5 * nz;
    double rnz = R6 * nx + R7 * ny + R8 * nz;
    const double rinv = 1.0 / smax(sqrt(rnx * rnx + rny * rny + rnz * rnz), 1e-12);
    rnx *= rinv;
    rny *= rinv;
    rnz *= rinv;

    ray_relu_ref(rnx, rny, rnz, rx, ry, rz, ox, oy, oz, pinv);
}

}  // namespace bvml
