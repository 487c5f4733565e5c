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

// one wave per row: 64 lanes x 8 k-values = the 512-d latent; the row's
// weights stay in registers while the frames are swept, one butterfly each.
__global__ __launch_bounds__(256) void style_gemv_kernel(const float *__restrict__ Wm,
                                                         const float *__restrict__ bm,
                                                         const float *__restrict__ lat,
                                                         float *__restrict__ s, SegTable seg,
                                                         int nframes) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int R = seg.row0[seg.n];
    if (row >= R) return;  // whole wave exits together
    const int sg = find_seg(seg, row);
    const int i = row - seg.row0[sg];
    const int width = seg.width[sg];
    float w[8];
    {
        const floatx4 a = *(const floatx4 *) (Wm + (int64_t) row * 512 + lane * 8);
        const floatx4 b = *(const floatx4 *) (Wm + (int64_t) row * 512 + lane * 8 + 4);
        w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
        w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
    }
    const float bias = bm[row];
    // the latents of FB frames are requested together, then reduced
    constexpr int FB = 8;
    for (int f0 = 0; f0 < nframes; f0 += FB) {
        floatx4 la[FB], lb[FB];
#pragma unroll
        for (int k = 0; k < FB; k++) {
            const int f = f0 + k < nframes ? f0 + k : nframes - 1;
            const float *l = lat + (int64_t) f * 512 + lane * 8;
            la[k] = *(const floatx4 *) l;
            lb[k] = *(const floatx4 *) (l + 4);
        }
#pragma unroll
        for (int k = 0; k < FB; k++) {
            const floatx4 a = la[k], b = lb[k];
            float acc = w[0] * a[0];
            acc = __builtin_fmaf(w[1], a[1], acc);
            acc = __builtin_fmaf(w[2], a[2], acc);
            acc = __builtin_fmaf(w[3], a[3], acc);
            acc = __builtin_fmaf(w[4], b[0], acc);
            acc = __builtin_fmaf(w[5], b[1], acc);
            acc = __builtin_fmaf(w[6], b[2], acc);
            acc = __builtin_fmaf(w[7], b[3], acc);
            acc = group_sum<64>(acc);
            if (lane == k && f0 + k < nframes) s[seg.out0[sg] + (int64_t) (f0 + k) * width + i] = acc + bias;
        }
    }
}

// one wave per (conv, output channel): den = sqrt(sum_i S[o][i] s_i^2 + S[o][IC]),
// FB frames at a time (each lane's partial sums over i = lane, lane+64, ...
// then the 64-lane butterfly, per frame)
__global__ __launch_bounds__(256) void demod_kernel(const float *__restrict__ saug,
                                                    const float *__restrict__ s,
                                                    float *__restrict__ inv_den, DemodTable t,
                                                    int nframes) {
#pragma clang fp contract(off)
    constexpr int FB = 8;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= t.row0[t.n]) return;
    int c = 0;
    while (c + 1 < t.n && row >= t.row0[c + 1]) c++;
    const int o = row - t.row0[c];
    const int IC = t.ic[c], OC = t.oc[c];
    const float *S = saug + t.saug0[c] + (int64_t) o * (IC + 1);
    // IC <= 512: the row's weights and each frame block's styles are all
    // requested before the first multiply-add (one memory round trip each)
    constexpr int JM = 8;
    const bool small = IC <= 64 * JM;
    float w[JM];
#pragma unroll
    for (int j = 0; j < JM; j++) w[j] = small && lane + 64 * j < IC ? S[lane + 64 * j] : 0.0f;
    for (int f0 = 0; f0 < nframes; f0 += FB) {
        float acc[FB];
#pragma unroll
        for (int k = 0; k < FB; k++) acc[k] = 0.0f;
        const float *sv = s + t.s0[c] + (int64_t) f0 * IC;
        if (small) {
            float sx[FB][JM];
#pragma unroll
            for (int k = 0; k < FB; k++)
#pragma unroll
                for (int j = 0; j < JM; j++)
                    sx[k][j] = f0 + k < nframes && lane + 64 * j < IC ? sv[(int64_t) k * IC + lane + 64 * j] : 0.0f;
#pragma unroll
            for (int k = 0; k < FB; k++)
#pragma unroll
                for (int j = 0; j < JM; j++) {
                    if (lane + 64 * j < IC) {
                        const float s2 = sx[k][j] * sx[k][j];
                        acc[k] = __builtin_fmaf(w[j], s2, acc[k]);
                    }
                }
        } else {
            for (int i = lane; i < IC; i += 64) {
                const float wi = S[i];
#pragma unroll
                for (int k = 0; k < FB; k++) {
                    if (f0 + k < nframes) {
                        const float si = sv[(int64_t) k * IC + i];
                        const float s2 = si * si;
                        acc[k] = __builtin_fmaf(wi, s2, acc[k]);
                    }
                }
            }
        }
        const float tail = S[IC];
#pragma unroll
        for (int k = 0; k < FB; k++) {
            const float sum = group_sum<64>(acc[k]);
            if (lane == k && f0 + k < nframes) {
                const float den = sqrtf(sum + tail);
                inv_den[t.d0[c] + (int64_t) (f0 + k) * OC + o] = 1.0f / den;
            }
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

hipError_t launch_style_gemv(const float *Wm, const float *bm, const float *lat, float *s,
                             const SegTable &seg, int nframes, hipStream_t st) {
    const int R = seg.row0[seg.n];
    if (R <= 0 || nframes <= 0) return hipSuccess;
    hipLaunchKernelGGL(style_gemv_kernel, dim3((R + 3) / 4), dim3(256), 0, st, Wm, bm, lat, s, seg,
                       nframes);
    return hipGetLastError();
}

hipError_t launch_demod(const float *saug, const float *s, float *inv_den, const DemodTable &t,
                        int nframes, hipStream_t st) {
    const int R = t.row0[t.n];
    if (R <= 0 || nframes <= 0) return hipSuccess;
    hipLaunchKernelGGL(demod_kernel, dim3((R + 3) / 4), dim3(256), 0, st, saug, s, inv_den, t,
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
