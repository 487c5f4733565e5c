// Bilinear grid-sample gather and the small per-pixel ops of the decoder's
// stage tail, as standalone kernels (the op-level surface of
// patches/ggml-tp-ops.patch: GGML_OP_BILINEAR_GATHER :683-752,
// GGML_OP_UPFIRDN2X :996-1045, GGML_OP_FLOW_GRID :1082-1104).
//
// The decoder itself runs these inside the fused stage-tail kernel
// (k_tail.hip); the standalone forms serve the op-level C ABI and tests.
#include "tpmd_device.h"
#include "tpmd_launch.h"

namespace tpmd {

// ---------------------------------------------------------------------------
// CL gather, vectorised: G lanes share one grid point and split its C
// channels in chunks of V = 4 elements (16 bytes f32, 8 bytes f16; CPL chunks
// per lane, C = G * CPL * 4).  All lanes of a group read the same tap rows,
// so a wave reads whole contiguous channel runs of the feature map
// (coalesced), and every lane writes one 16-byte f32 vector per chunk, so
// each store instruction covers a contiguous run of the output row.
//
// Each lane group takes P points per pass and issues all 4 * P * CPL tap
// loads before it consumes any, so a wave keeps that many loads in flight
// instead of waiting on one tap at a time.  The taps are read through a
// buffer resource that spans the feature map: a tap outside the map gets an
// offset past the end, which the hardware answers with zeros, and its weight
// is set to zero, so it adds +0 to the sum, which leaves the sum bitwise as
// it is when the tap is skipped (the sum starts at +0 and a round-to-nearest
// sum is -0 only when both terms are).  The output is written once and not
// read again here: non-temporal stores.  (Measured on MI355X at C = 32..512,
// 16 frames: 8-byte f16 chunks with non-temporal stores beat 16-byte chunks,
// whose two stores per lane each cover every other 16 bytes of a row, by up
// to 2x; a grid of 4096 blocks, 16 per CU, looping over the points, beats
// one pass per wave by up to 10 %, and P = 1 is on par with P = 2 and 4.)
//
// NS = 4 (maps of 8 MB or more, twice an XCD's 4 MB L2, with rows of at
// least 1 KB): the channels split into 4 slices; workgroup b runs on XCD
// b % 8 and takes slice b % 4 of every point, so each XCD's L2 holds a
// quarter of the feature map (2 MB of a 512-channel f32 64 x 64 map) and the
// random taps of an i.i.d. grid hit it instead of going to HBM.  The sums are
// the same per element, so the result is bitwise the NS = 1 one.  (Measured
// on MI355X, 512 x 64 x 64 f32, 16 frames of i.i.d. taps: 52.6 us unsliced,
// 34.2 us with 8 slices, 32.5 us with 4; two points per lane group in flight
// are slower with either.)
constexpr uint32_t kTapOutside = 0x80000000u;  // past any feature map this kernel accepts

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// V elements of TF at byte offset off of the buffer (zeros past its end)
template <typename TF, int V> struct tap_chunk;
template <> struct tap_chunk<float, 4> {
    typedef floatx4 type;
    static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
        return __builtin_bit_cast(type, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
};
template <> struct tap_chunk<half_t, 4> {
    typedef half4 type;
    static __device__ __forceinline__ type load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
        return __builtin_bit_cast(type, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
    }
};
template <typename TF, int V, int G, int CPL, int P, int NS>
__global__ __launch_bounds__(256) void gather_cl_vec(const TF *__restrict__ feat, uint32_t feat_bytes,
                                                     const float *__restrict__ grid,
                                                     float *__restrict__ dst, int C, int W, int H,
                                                     int64_t N, int planar) {
#pragma clang fp contract(off)
    typedef tap_chunk<TF, V> ld;
    typedef typename ld::type vt;
    constexpr int CB = V * (int) sizeof(TF);  // bytes per chunk
    constexpr int PPW = 64 / G;               // points per wave and pass
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *) feat, (short) 0, (int) feat_bytes, 0x00020000);
    const int lane = threadIdx.x & 63;
    const int gl = lane % G, grp = lane / G;
    const uint32_t row_bytes = (uint32_t) C * sizeof(TF);
    // channel slice of this workgroup (its XCD) and its place among the
    // workgroups of that slice
    const int slice = NS > 1 ? (int) (blockIdx.x % NS) : 0;
    const int64_t blk = NS > 1 ? (int64_t) (blockIdx.x / NS) : (int64_t) blockIdx.x;
    const int64_t nblk = NS > 1 ? (int64_t) (gridDim.x / NS) : (int64_t) gridDim.x;
    const int cs = slice * (C / NS);          // first channel of the slice
    const int64_t wave = blk * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nwaves = nblk * (blockDim.x >> 6);
    for (int64_t n0 = wave * PPW * P + grp; n0 < N; n0 += nwaves * PPW * P) {
        uint32_t off[P][4];
        float w[P][4];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int64_t n = n0 + p * PPW < N ? n0 + p * PPW : N - 1;
            const float gx = planar ? grid[n] : grid[2 * n];
            const float gy = planar ? grid[N + n] : grid[2 * n + 1];
            const taps4 t = gather_geometry(gx, gy, W, H);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const bool in = tap_inside(t, k, W, H);
                off[p][k] = in ? (uint32_t) ((t.y0 + (k >> 1)) * W + t.x0 + (k & 1)) * row_bytes +
                                     (uint32_t) (cs * (int) sizeof(TF)) + gl * CB
                               : kTapOutside;
                w[p][k] = in ? tap_weight(t, k) : 0.0f;
            }
        }
        vt v[P][4][CPL];
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int k = 0; k < 4; k++)
#pragma unroll
                for (int ch = 0; ch < CPL; ch++) v[p][k][ch] = ld::load(rs, off[p][k] + ch * G * CB);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int64_t n = n0 + p * PPW;
            if (n >= N) break;
            float *d = dst + n * C + cs;
#pragma unroll
            for (int ch = 0; ch < CPL; ch++) {
                float acc[V];
#pragma unroll
                for (int e = 0; e < V; e++) acc[e] = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; k++)
#pragma unroll
                    for (int e = 0; e < V; e++) acc[e] += w[p][k] * to_f32(v[p][k][ch][e]);
                float *dd = d + (ch * G + gl) * V;
#pragma unroll
                for (int e = 0; e < V; e += 4) {
                    __builtin_nontemporal_store(floatx4{acc[e], acc[e + 1], acc[e + 2], acc[e + 3]},
                                                (floatx4 *) (dd + e));
                }
            }
        }
    }
}

// one thread per output element (any C, CL or SP output): the layout- and
// size-generic form, mirroring the reference kernel's indexing
template <typename TF>
__global__ __launch_bounds__(256) void gather_elem(const TF *__restrict__ feat,
                                                   const float *__restrict__ grid,
                                                   float *__restrict__ dst, int C, int W, int H,
                                                   int64_t N, int planar, int sp) {
#pragma clang fp contract(off)
    const int64_t total = (int64_t) C * N;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int c = sp ? (int) (i / N) : (int) (i % C);
        const int64_t n = sp ? i % N : i / C;
        const float gx = planar ? grid[n] : grid[2 * n];
        const float gy = planar ? grid[N + n] : grid[2 * n + 1];
        const taps4 t = gather_geometry(gx, gy, W, H);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (!tap_inside(t, k, W, H)) continue;
            const int cx = t.x0 + (k & 1), cy = t.y0 + (k >> 1);
            acc += tap_weight(t, k) * to_f32(feat[(int64_t) (cy * W + cx) * C + c]);
        }
        dst[i] = acc;
    }
}

// integer tap selection and f32 weights per point
__global__ __launch_bounds__(256) void gather_taps_kernel(const float *__restrict__ grid, int W,
                                                          int H, int64_t N, int planar,
                                                          int32_t *__restrict__ x0,
                                                          int32_t *__restrict__ y0,
                                                          float *__restrict__ wx,
                                                          float *__restrict__ wy) {
    for (int64_t n = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; n < N;
         n += (int64_t) gridDim.x * blockDim.x) {
        const float gx = planar ? grid[n] : grid[2 * n];
        const float gy = planar ? grid[N + n] : grid[2 * n + 1];
        const taps4 t = gather_geometry(gx, gy, W, H);
        x0[n] = t.x0;
        y0[n] = t.y0;
        wx[n] = t.wx;
        wy[n] = t.wy;
    }
}

// upfirdn2d(up=2, pad=(2,1)): SP [CB][H][W] -> [CB][2H][2W]
__global__ __launch_bounds__(256) void upfirdn2x_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ k4,
                                                        float *__restrict__ y, int W, int H,
                                                        int64_t CB) {
    const int64_t total = 4 * (int64_t) W * H * CB;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int X = (int) (i % (2 * W));
        const int Y = (int) ((i / (2 * W)) % (2 * H));
        const int64_t cb = i / (4 * (int64_t) W * H);
        y[i] = upfirdn2x_at(x + (int64_t) W * H * cb, W, H, k4, X, Y);
    }
}

// flow head: fl SP [3][N], xs planar [2][N] -> [3][N] (gx, gy, mask)
__global__ __launch_bounds__(256) void flow_grid_kernel(const float *__restrict__ fl,
                                                        const float *__restrict__ xs,
                                                        float *__restrict__ y, int64_t N) {
#pragma clang fp contract(off)
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < 3 * N;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t pln = i / N, n = i % N;
        y[i] = pln == 2 ? 1.0f / (1.0f + expf(-fl[2 * N + n])) : tanhf(fl[pln * N + n]) + xs[pln * N + n];
    }
}

// CHW f32 frames in [-1, 1] -> interleaved 8-bit RGB, the video writer's
// conversion (tools/tp-cli.cpp:43-53): clamp to [-1, 1], (v + 1) / 2 * 255,
// truncated toward zero.  Four pixels per thread: float4 reads of each
// plane, three 32-bit stores of the 12 interleaved bytes.
__global__ __launch_bounds__(256) void rgb24_kernel(const float *__restrict__ chw,
                                                    uint8_t *__restrict__ rgb, int n, int R) {
#pragma clang fp contract(off)
    const int64_t quads = (int64_t) R * R / 4;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < quads * n;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int64_t f = i / quads, q = i - f * quads;
        const float *src = chw + f * 3 * (int64_t) R * R + q * 4;
        uint8_t b[12];
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const floatx4 v = *(const floatx4 *) (src + (int64_t) c * R * R);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float x = v[e];
                x = x < -1.0f ? -1.0f : (x > 1.0f ? 1.0f : x);
                b[e * 3 + c] = (uint8_t) ((x + 1.0f) / 2.0f * 255.0f);
            }
        }
        uint32_t w[3];
        __builtin_memcpy(w, b, 12);
        uint32_t *dst = (uint32_t *) (rgb + (f * (int64_t) R * R + q * 4) * 3);
        dst[0] = w[0];
        dst[1] = w[1];
        dst[2] = w[2];
    }
}

// ---------------------------------------------------------------------------
// launchers

static int grid_for(int64_t work, int per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (int) g;
}

template <typename TF>
static hipError_t launch_gather_typed(const TF *feat, const float *grid, float *dst, int C, int W,
                                      int H, int64_t N, int planar, int sp, hipStream_t st) {
    constexpr int VEC = 4;
    const bool aligned = (((uintptr_t) feat | (uintptr_t) dst) & 15) == 0;
    const int64_t feat_bytes = (int64_t) W * H * C * (int64_t) sizeof(TF);
    if (!sp && C % VEC == 0 && aligned && feat_bytes < (int64_t) kTapOutside) {
        // a map of 8 MB or more (twice an XCD's L2) with rows of 1 KB or
        // more: one channel slice per XCD
        const int NS = feat_bytes >= (8 << 20) && (int64_t) C * (int64_t) sizeof(TF) >= 1024 &&
                               C % (4 * VEC) == 0 ? 4 : 1;
        const int lpp = C / NS / VEC;
        int G = 0, CPL = 0;
        if (lpp <= 64 && (lpp & (lpp - 1)) == 0) {
            G = lpp;
            CPL = 1;
        } else if (lpp % 64 == 0 && (lpp / 64 == 2 || lpp / 64 == 4 || lpp / 64 == 8)) {
            G = 64;
            CPL = lpp / 64;
        }
        if (G) {
            constexpr int P = 1;
            int nb = grid_for(N, 4 * (64 / G) * P);  // 4 waves per 256-thread block, per slice
            if (nb > 4096 / NS) nb = 4096 / NS;
            nb *= NS;
#define TPMD_G(g, cpl, p, ns)                                                                         \
    if (G == g && CPL == cpl && P == p && NS == ns) {                                                           \
        hipLaunchKernelGGL((gather_cl_vec<TF, VEC, g, cpl, p, ns>), dim3(nb), dim3(256), 0, st, feat, \
                           (uint32_t) feat_bytes, grid, dst, C, W, H, N, planar);                    \
        return hipGetLastError();                                                                     \
    }
            TPMD_G(1, 1, 1, 1) TPMD_G(2, 1, 1, 1) TPMD_G(4, 1, 1, 1) TPMD_G(8, 1, 1, 1) TPMD_G(16, 1, 1, 1)
            TPMD_G(32, 1, 1, 1) TPMD_G(64, 1, 1, 1) TPMD_G(64, 2, 1, 1) TPMD_G(64, 4, 1, 1) TPMD_G(64, 8, 1, 1)
            TPMD_G(16, 1, 1, 4) TPMD_G(32, 1, 1, 4) TPMD_G(64, 1, 1, 4)
            TPMD_G(64, 2, 1, 4) TPMD_G(64, 4, 1, 4) TPMD_G(64, 8, 1, 4)
#undef TPMD_G
        }
    }
    hipLaunchKernelGGL((gather_elem<TF>), dim3(grid_for((int64_t) C * N, 256)), dim3(256), 0, st,
                       feat, grid, dst, C, W, H, N, planar, sp);
    return hipGetLastError();
}

hipError_t launch_gather(const void *feat, bool feat_f16, const float *grid, float *dst, int C,
                         int W, int H, int64_t N, int planar, int sp, hipStream_t st) {
    if (N <= 0 || C <= 0) return hipSuccess;
    if (feat_f16)
        return launch_gather_typed((const half_t *) feat, grid, dst, C, W, H, N, planar, sp, st);
    return launch_gather_typed((const float *) feat, grid, dst, C, W, H, N, planar, sp, st);
}

hipError_t launch_gather_taps(const float *grid, int W, int H, int64_t N, int planar, int32_t *x0,
                              int32_t *y0, float *wx, float *wy, hipStream_t st) {
    if (N <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_taps_kernel, dim3(grid_for(N, 256)), dim3(256), 0, st, grid, W, H,
                       N, planar, x0, y0, wx, wy);
    return hipGetLastError();
}

hipError_t launch_upfirdn2x(const float *x, const float *k4, float *y, int W, int H, int64_t CB,
                            hipStream_t st) {
    if (CB <= 0 || W <= 0 || H <= 0) return hipSuccess;
    hipLaunchKernelGGL(upfirdn2x_kernel, dim3(grid_for(4 * (int64_t) W * H * CB, 256)), dim3(256),
                       0, st, x, k4, y, W, H, CB);
    return hipGetLastError();
}

hipError_t launch_rgb24(const float *chw, int n, int R, uint8_t *rgb, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(rgb24_kernel, dim3(grid_for((int64_t) n * R * R / 4, 256)), dim3(256), 0, st, chw, rgb,
                       n, R);
    return hipGetLastError();
}

hipError_t launch_flow_grid(const float *fl, const float *xs, float *y, int64_t N,
                            hipStream_t st) {
    if (N <= 0) return hipSuccess;
    hipLaunchKernelGGL(flow_grid_kernel, dim3(grid_for(3 * N, 256)), dim3(256), 0, st, fl, xs, y,
                       N);
    return hipGetLastError();
}

}  // namespace tpmd
