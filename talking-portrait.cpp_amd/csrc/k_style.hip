// Per-frame style work of one decode batch (src/motion_dec.cpp:267-280,
// :375-393):
//   style  s_L = Wmod_L . w + bmod_L          every modulated conv L (one launch)
//   demod  1/den_L, den_L = sqrt(S_aug_L . [s_L^2; 1])   every demod conv (one launch)
//   conv1  input (4x4 constant) * s_conv1 in the conv operand type (one launch)
// Rows of all convs are concatenated; a small table maps a global row to its
// conv, and each conv's outputs are stored [frame][channel] contiguously.
#include "tpmd_device.h"
#include "tpmd_launch.h"

namespace tpmd {

__device__ __forceinline__ int find_seg(const SegTable &t, int row) {
    int s = 0;
    while (s + 1 < t.n && row >= t.row0[s + 1]) s++;
    return s;
}

// Both are skinny GEMMs, Y[f][row] = sum_k W[row][k] X[f][k] over 16 frames,
// run on v_mfma_f32_16x16x4_f32: a wave computes 16 rows x 16 frames.  Lane l
// feeds A = W[row0 + l%16][k] and B = X[f0 + l%16][k] for k = kb + 4(l/16) + j,
// j = 0..3 (one MFMA each: a 16-byte load per operand covers four k steps,
// the k order inside a 16-wide block permuted the same way for both); the
// result of lane l, element v is row row0 + 4(l/16) + v, frame f0 + l%16.
// A frame's sums never mix with another frame's (its own MFMA column).
__device__ __forceinline__ floatx4 mfma16x4_block(const floatx4 a, const floatx4 b, floatx4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
    return acc;
}

// Both run one 16-row tile per workgroup with the k range split over its
// four waves (quarters of the 16-wide k blocks, in order): a wave streams a
// quarter of the tile's row of W, so the tile's loads are in flight together
// instead of one wave walking all of K; the four partial tiles are added in
// wave order through LDS (the same sums for every batch).
__device__ __forceinline__ floatx4 ksplit_sum(floatx4 acc, int wid, int lane) {
    __shared__ floatx4 part[3][64];
    if (wid > 0) part[wid - 1][lane] = acc;
    __syncthreads();
    if (wid == 0) {
#pragma unroll
        for (int w = 0; w < 3; w++) {
            const floatx4 b = part[w][lane];
#pragma unroll
            for (int j = 0; j < 4; j++) acc[j] = acc[j] + b[j];
        }
    }
    return acc;
}

// style: W = Wmod (all convs' rows, K = 512), X = the latents
__global__ __launch_bounds__(256) void style_gemv_kernel(const float *__restrict__ Wm,
                                                         const float *__restrict__ bm,
                                                         const float *__restrict__ lat,
                                                         float *__restrict__ s, SegTable seg,
                                                         int nframes) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 16;
    const int sg = find_seg(seg, r0);
    const int li = lane & 15, kq = lane >> 4;
    const int f0 = blockIdx.y * 16;
    const int f = f0 + li < nframes ? f0 + li : nframes - 1;
    const int k0 = wid * 128;
    const float *wp = Wm + (int64_t) (r0 + li) * 512 + k0 + kq * 4;
    const float *xp = lat + (int64_t) f * 512 + k0 + kq * 4;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 128; kb += 16)
        acc = mfma16x4_block(*(const floatx4 *) (wp + kb), *(const floatx4 *) (xp + kb), acc);
    acc = ksplit_sum(acc, wid, lane);
    if (wid == 0 && f0 + li < nframes) {
        const int width = seg.width[sg];
        float *out = s + seg.out0[sg] + (int64_t) (f0 + li) * width + (r0 - seg.row0[sg]) + kq * 4;
#pragma unroll
        for (int v = 0; v < 4; v++) out[v] = acc[v] + bm[r0 + kq * 4 + v];
    }
}

// demod: den = sqrt(sum_i S[o][i] s_i^2 + S_tail[o]) per (demod conv, output
// channel o), W = S_aug rows of the conv, X = its styles squared
__global__ __launch_bounds__(256) void demod_kernel(const float *__restrict__ saug,
                                                    const float *__restrict__ s,
                                                    float *__restrict__ inv_den, DemodTable t,
                                                    int nframes) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 16;
    int c = 0;
    while (c + 1 < t.n && r0 >= t.row0[c + 1]) c++;
    const int o0 = r0 - t.row0[c];
    const int IC = t.ic[c], OC = t.oc[c];
    const float *S = saug + t.saug0[c];
    const int li = lane & 15, kq = lane >> 4;
    const int f0 = blockIdx.y * 16;
    const int f = f0 + li < nframes ? f0 + li : nframes - 1;
    // this wave's quarter of the IC / 16 k blocks
    const int nb = IC / 16, kb0 = (wid * nb) / 4 * 16, kb1 = ((wid + 1) * nb) / 4 * 16;
    const float *wp = S + (int64_t) (o0 + li) * IC + kq * 4;
    const float *xp = s + t.s0[c] + (int64_t) f * IC + kq * 4;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int kb = kb0; kb < kb1; kb += 16) {
        const floatx4 x = *(const floatx4 *) (xp + kb);
        floatx4 x2;
#pragma unroll
        for (int j = 0; j < 4; j++) x2[j] = x[j] * x[j];
        acc = mfma16x4_block(*(const floatx4 *) (wp + kb), x2, acc);
    }
    acc = ksplit_sum(acc, wid, lane);
    if (wid == 0 && f0 + li < nframes) {
        float *out = inv_den + t.d0[c] + (int64_t) (f0 + li) * OC + o0 + kq * 4;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float den = sqrtf(acc[v] + S[(int64_t) OC * IC + o0 + kq * 4 + v]);
            out[v] = 1.0f / den;
        }
    }
}

// xs0[f][p][c] = act(in[p][c] * s[f][c]), p < 16
template <typename TA>
__global__ __launch_bounds__(256) void prescale_input_kernel(const float *__restrict__ in,
                                                             const float *__restrict__ s,
                                                             TA *__restrict__ xs, int C,
                                                             int nframes) {
    const int64_t total = (int64_t) nframes * 16 * C;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int c = (int) (i % C);
        const int64_t f = i / (16 * C);
        const int p = (int) ((i / C) % 16);
        xs[i] = from_f32<TA>(in[p * C + c] * s[f * C + c]);
    }
}

// x[f][p][c] -> act(x * s[f][c]) (f32 input maps, test entry points)
template <typename TA>
__global__ __launch_bounds__(256) void prescale_map_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ s,
                                                           TA *__restrict__ xs, int C,
                                                           int64_t npix_per_frame,
                                                           int64_t total) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t) gridDim.x * blockDim.x) {
        const int c = (int) (i % C);
        const int64_t f = i / (npix_per_frame * C);
        xs[i] = from_f32<TA>(x[i] * (s ? s[f * C + c] : 1.0f));
    }
}

// 16-row tiles: every segment starts and ends on a multiple of 16 rows
hipError_t launch_style_gemv(const float *Wm, const float *bm, const float *lat, float *s,
                             const SegTable &seg, int nframes, hipStream_t st) {
    const int R = seg.row0[seg.n];
    if (R <= 0 || nframes <= 0) return hipSuccess;
    for (int i = 0; i <= seg.n; i++)
        if (seg.row0[i] % 16 != 0) return hipErrorInvalidValue;
    const int tiles = R / 16;
    hipLaunchKernelGGL(style_gemv_kernel, dim3(tiles, (nframes + 15) / 16), dim3(256), 0, st, Wm, bm, lat, s, seg,
                       nframes);
    return hipGetLastError();
}

hipError_t launch_demod(const float *saug, const float *s, float *inv_den, const DemodTable &t,
                        int nframes, hipStream_t st) {
    const int R = t.row0[t.n];
    if (R <= 0 || nframes <= 0) return hipSuccess;
    for (int i = 0; i < t.n; i++)
        if (t.row0[i] % 16 != 0 || t.ic[i] % 16 != 0 || t.oc[i] % 16 != 0 || t.saug0[i] % 4 != 0 ||
            t.s0[i] % 4 != 0)
            return hipErrorInvalidValue;
    const int tiles = R / 16;
    hipLaunchKernelGGL(demod_kernel, dim3(tiles, (nframes + 15) / 16), dim3(256), 0, st, saug, s, inv_den, t,
                       nframes);
    return hipGetLastError();
}

hipError_t launch_prescale_input(bool f16, const float *in, const float *s, void *xs, int C,
                                 int nframes, hipStream_t st) {
    const int64_t total = (int64_t) nframes * 16 * C;
    if (total <= 0) return hipSuccess;
    const int nb = (int) ((total + 255) / 256 > 4096 ? 4096 : (total + 255) / 256);
    if (f16)
        hipLaunchKernelGGL((prescale_input_kernel<half_t>), dim3(nb), dim3(256), 0, st, in, s,
                           (half_t *) xs, C, nframes);
    else
        hipLaunchKernelGGL((prescale_input_kernel<float>), dim3(nb), dim3(256), 0, st, in, s,
                           (float *) xs, C, nframes);
    return hipGetLastError();
}

hipError_t launch_prescale_map(bool f16, const float *x, const float *s, void *xs, int C,
                               int64_t npix_per_frame, int nframes, hipStream_t st) {
    const int64_t total = (int64_t) nframes * npix_per_frame * C;
    if (total <= 0) return hipSuccess;
    const int nb = (int) ((total + 255) / 256 > 65536 ? 65536 : (total + 255) / 256);
    if (f16)
        hipLaunchKernelGGL((prescale_map_kernel<half_t>), dim3(nb), dim3(256), 0, st, x, s,
                           (half_t *) xs, C, npix_per_frame, total);
    else
        hipLaunchKernelGGL((prescale_map_kernel<float>), dim3(nb), dim3(256), 0, st, x, s,
                           (float *) xs, C, npix_per_frame, total);
    return hipGetLastError();
}

}  // namespace tpmd
