// Device-side building blocks shared by the motion-decoder kernels (gfx950).
//
// Conventions:
//   * activations are channel-last ("CL"): [frame][y][x][channel], the
//     channel dimension contiguous, matching the reference's [C, N, B]
//     fast-graph layout (src/motion_dec.cpp:240-241);
//   * skip pyramids (rgb, flow) are per-frame planes [frame][3][y][x] f32,
//     the reference's spatial [W, H, 3, B] layout;
//   * "act_t" is the storage type of conv operands: _Float16 in f16 mode
//     (f16 in, f32 accumulate), float in f32 mode.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tpmd {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kSlope = 0.2f;

// v > 0 ? v : 0.2 v, as one max: for v > 0, v > 0.2 v; otherwise 0.2 v >= v
// (and both zeros and infinities come out as the select gives them)
__device__ __forceinline__ float leaky(float v) { return __builtin_fmaxf(v, kSlope * v); }

// 16-byte vector of act_t and its element count
template <typename T> struct vec16;
template <> struct vec16<float> {
    typedef floatx4 type;
    static constexpr int n = 4;
};
template <> struct vec16<half_t> {
    typedef half8 type;
    static constexpr int n = 8;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(half_t v) { return (float) v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ half_t from_f32<half_t>(float v) { return (half_t) v; }

// v of the lane `lane ^ M` (M a power of two < 64): DPP quad permutes for
// M = 1, 2 (no LDS traffic), ds_swizzle bit-masks for M = 4, 8, 16 (within
// 32 lanes, no LDS addressing), ds_bpermute for M = 32
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __builtin_bit_cast(int, v);
    int y;
    if constexpr (M == 1) y = __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);       // [1,0,3,2]
    else if constexpr (M == 2) y = __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // [2,3,0,1]
    else if constexpr (M < 32) y = __builtin_amdgcn_ds_swizzle(x, 0x1F | (M << 10));
    else y = __builtin_bit_cast(int, __shfl_xor(v, M, 64));
    return __builtin_bit_cast(float, y);
}

// sum over aligned groups of G lanes (G a power of two <= 64), result in
// every lane of the group: xor butterfly, each step adding the partner's
// value to the lane's own (so every lane ends with the same bits)
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += lane_xor<1>(v);
    if constexpr (G >= 4) v += lane_xor<2>(v);
    if constexpr (G >= 8) v += lane_xor<4>(v);
    if constexpr (G >= 16) v += lane_xor<8>(v);
    if constexpr (G >= 32) v += lane_xor<16>(v);
    if constexpr (G >= 64) v += lane_xor<32>(v);
    return v;
}

// upfirdn2d(up=2, pad=(2,1)) of one SP plane at output (X, Y), 4x4 kernel
// k4[i + 4j] (patch :996-1018 semantics).  Of the 4x4 window over the
// zero-stuffed map, only taps with X+i-2 and Y+j-2 even hit a source pixel:
// i in {X&1, X&1 + 2}, j in {Y&1, Y&1 + 2}, i.e. source columns
// (X + (X&1) - 2)/2 + {0, 1} and the same for rows.  They are visited in
// the reference loop's order (j-major, i-minor, out-of-map taps skipped), so
// the sum equals the 16-tap loop's bit for bit.  The four loads use clamped
// (always in-map) indices; an out-of-map tap leaves the sum as it was,
// exactly as skipping it does.  Split in two so that a caller can request the
// taps of several planes before summing any of them.
struct upfirdn_taps {
    float v[4], k[4];
    bool in[4];
};
__device__ __forceinline__ void upfirdn2x_load(const float *__restrict__ plane, int W, int H,
                                               const float *__restrict__ k4, int X, int Y, upfirdn_taps &t) {
    const int i0 = X & 1, j0 = Y & 1;
    const int sx0 = (X + i0 - 2) >> 1, sy0 = (Y + j0 - 2) >> 1;
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
        const int sy = sy0 + jj;
        const int cy = sy < 0 ? 0 : (sy >= H ? H - 1 : sy);
#pragma unroll
        for (int ii = 0; ii < 2; ii++) {
            const int sx = sx0 + ii;
            const int cx = sx < 0 ? 0 : (sx >= W ? W - 1 : sx);
            t.in[2 * jj + ii] = (unsigned) sy < (unsigned) H && (unsigned) sx < (unsigned) W;
            t.v[2 * jj + ii] = plane[cx + W * cy];
            t.k[2 * jj + ii] = k4[i0 + 2 * ii + 4 * (j0 + 2 * jj)];
        }
    }
}
// the four kernel taps output (X, Y) uses, in upfirdn_taps order: the 16
// taps are the same for every lane (scalar loads), the lane's four follow
// from its output parity by selects, so planes that share the kernel share
// them and no lane issues a vector load for a weight
struct upfirdn_k {
    float k[4];
};
__device__ __forceinline__ upfirdn_k upfirdn2x_weights(const float *__restrict__ k4, int X, int Y) {
    // (read through the constant address space: a uniform address there is
    // a scalar load; the kernel is never written while a launch runs.  The
    // taps are named values, not an array, and pass through readfirstlane,
    // so the selects stay register selects instead of being folded into an
    // indexed private array)
    const __attribute__((address_space(4))) float *kc = (const __attribute__((address_space(4))) float *) k4;
    auto sk = [&](int q) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(kc[q]))); };
    const float k0 = sk(0), k1 = sk(1), k2 = sk(2), k3 = sk(3), k4_ = sk(4), k5 = sk(5), k6 = sk(6), k7 = sk(7);
    const float k8 = sk(8), k9 = sk(9), k10 = sk(10), k11 = sk(11), k12 = sk(12), k13 = sk(13), k14 = sk(14),
                k15 = sk(15);
    const bool i1 = X & 1, j1 = Y & 1;
    // tap (ii, jj) is k4[i0 + 2*ii + 4*(j0 + 2*jj)]: of b, b+1, b+4, b+5 with b = 2*ii + 8*jj
    auto pick = [&](float kb, float kb1, float kb4, float kb5) { return j1 ? (i1 ? kb5 : kb4) : (i1 ? kb1 : kb); };
    upfirdn_k r;
    r.k[0] = pick(k0, k1, k4_, k5);
    r.k[1] = pick(k2, k3, k6, k7);
    r.k[2] = pick(k8, k9, k12, k13);
    r.k[3] = pick(k10, k11, k14, k15);
    return r;
}
// the data taps read through a buffer resource over the whole skip array:
// plane0 = the plane's first element, 32-bit offsets instead of a 64-bit
// address per tap; the kernel taps from upfirdn2x_weights
__device__ __forceinline__ void upfirdn2x_load(__amdgpu_buffer_rsrc_t rs, unsigned plane0, int W, int H,
                                               const upfirdn_k &kw, int X, int Y, upfirdn_taps &t) {
    const int i0 = X & 1, j0 = Y & 1;
    const int sx0 = (X + i0 - 2) >> 1, sy0 = (Y + j0 - 2) >> 1;
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
        const int sy = sy0 + jj;
        const int cy = sy < 0 ? 0 : (sy >= H ? H - 1 : sy);
#pragma unroll
        for (int ii = 0; ii < 2; ii++) {
            const int sx = sx0 + ii;
            const int cx = sx < 0 ? 0 : (sx >= W ? W - 1 : sx);
            t.in[2 * jj + ii] = (unsigned) sy < (unsigned) H && (unsigned) sx < (unsigned) W;
            t.v[2 * jj + ii] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rs, (plane0 + (unsigned) (cx + W * cy)) * 4u, 0, 0));
            t.k[2 * jj + ii] = kw.k[2 * jj + ii];
        }
    }
}

// p[i] for a uniform p and i as a scalar load (through the constant address
// space; the data is never written while a launch runs), kept a register
// value by readfirstlane so that selects between such values are not folded
// into a vector load at a per-lane address
__device__ __forceinline__ float ld_uniform(const float *p, int i) {
    const __attribute__((address_space(4))) float *c = (const __attribute__((address_space(4))) float *) p;
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(c[i])));
}

// buffer resource over `bytes` bytes at p (bytes < 2^31)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *) p, (short) 0, (int) bytes, 0x00020000);
}

__device__ __forceinline__ float upfirdn2x_sum(const upfirdn_taps &t) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {  // j-major, i-minor
        const float s = acc + t.v[q] * t.k[q];
        acc = t.in[q] ? s : acc;
    }
    return acc;
}
__device__ __forceinline__ float upfirdn2x_at(const float *__restrict__ plane, int W, int H,
                                              const float *__restrict__ k4, int X, int Y) {
    upfirdn_taps t;
    upfirdn2x_load(plane, W, H, k4, X, Y, t);
    return upfirdn2x_sum(t);
}

// grid_sample (bilinear, zeros, align_corners=False) tap geometry for one
// point, computed with one rounding per operation (patch :688-718):
//   fx = (gx + 1) * 0.5 * W - 0.5,  x0 = floor(fx),  wx = fx - x0
struct taps4 {
    int x0, y0;
    float wx, wy;
};
__device__ __forceinline__ taps4 gather_geometry(float gx, float gy, int W, int H) {
#pragma clang fp contract(off)
    taps4 t;
    const float fx = (gx + 1.0f) * 0.5f * (float) W - 0.5f;
    const float fy = (gy + 1.0f) * 0.5f * (float) H - 0.5f;
    const float fxf = floorf(fx), fyf = floorf(fy);
    t.x0 = (int) fxf;
    t.y0 = (int) fyf;
    t.wx = fx - fxf;
    t.wy = fy - fyf;
    return t;
}

// tap k (cx = x0 + (k&1), cy = y0 + (k>>1)) lies inside the W x H map.
// Written without forming x0 + 1: an infinite coordinate converts to
// INT_MAX / INT_MIN, and x0 + 1 would wrap into the map.
__device__ __forceinline__ bool tap_inside(const taps4 &t, int k, int W, int H) {
    const int dx = k & 1, dy = k >> 1;
    return t.x0 >= -dx && t.x0 < W - dx && t.y0 >= -dy && t.y0 < H - dy;
}

// weight of tap k (cx = x0 + (k&1), cy = y0 + (k>>1))
__device__ __forceinline__ float tap_weight(const taps4 &t, int k) {
#pragma clang fp contract(off)
    return ((k & 1) ? t.wx : 1.0f - t.wx) * ((k >> 1) ? t.wy : 1.0f - t.wy);
}

}  // namespace tpmd
