/*
 * CPU ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the arithmetic of talking-portrait.cpp's motion
 * decoder (src/motion_dec.cpp) and of the custom ggml ops it is built from
 * (patches/ggml-tp-ops.patch, CPU kernels :308-657).  It exists to CHECK the
 * HIP implementation; the shipped library never links, loads or calls it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Built with -ffp-contract=off so every float expression below rounds once
 * per operation, exactly as written (no fused multiply-add anywhere).
 *
 * Layout vocabulary (ggml "ne" order, fastest first):
 *   CL  = [C, N, B]      channel-fastest maps, N = x + W*y
 *   SP  = [W, H, C, B]   plane-per-channel maps (torch NCHW)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* IEEE binary16 round-to-nearest-even (the rounding ggml_fp32_to_fp16
 * applies on F16C hosts and __float2half applies on GPUs).             */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t) (sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* result is subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t) sign; /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23;                /* 102..112 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;            /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t) (sign | r);
    }
    /* normal range: rebias exponent 127 -> 15 and round 13 mantissa bits */
    uint32_t r = (ax - 0x38000000u) >> 13;
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t) (sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float) m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* in-place round of an f32 array to f16-representable values */
void orc_round_f16(float *x, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) x[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
}

void orc_to_f16_bits(const float *x, uint16_t *h, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) h[i] = orc_f32_to_f16(x[i]);
}

/* ------------------------------------------------------------------ */
/* prepare(): derived tensors (src/motion_dec.cpp:104-223).
 * W is the scale-folded f32 host copy in torch order [OC][IC][3][3].    */

/* S_aug [OC][IC+1]: 0.5 * sum_k W^2 (double accumulation -> f32), last
 * column 0.5e-8  (src/motion_dec.cpp:113-122) */
void orc_saug(const float *W, int OC, int IC, int KK, float *out) {
#pragma omp parallel for schedule(static)
    for (int o = 0; o < OC; o++) {
        for (int i = 0; i < IC; i++) {
            double s = 0;
            const float *pw = W + ((size_t) o * IC + i) * KK;
            for (int k = 0; k < KK; k++) s += (double) pw[k] * pw[k];
            out[(size_t) o * (IC + 1) + i] = (float) (s * 0.5);
        }
        out[(size_t) o * (IC + 1) + IC] = 0.5e-8f;
    }
}

/* dense cf GEMM matrix A_cf[o][r], r = ic + IC*(kw + 3*kh)
 * (src/motion_dec.cpp:132-143) */
void orc_acf(const float *W, int OC, int IC, float *out) {
    const size_t R = (size_t) IC * 9;
#pragma omp parallel for schedule(static)
    for (int o = 0; o < OC; o++)
        for (int i = 0; i < IC; i++)
            for (int kh = 0; kh < 3; kh++)
                for (int kw = 0; kw < 3; kw++)
                    out[(size_t) o * R + i + (size_t) IC * (kw + 3 * kh)] =
                        W[((size_t) o * IC + i) * 9 + kh * 3 + kw];
}

/* conv_transpose(3x3, s2) o Blur(4x4) composed per output parity class
 * (by,bx) into a 3x3 pad-1 kernel (src/motion_dec.cpp:144-186):
 *   T[ty][tx] = sum_{cy,cx} V[cy][cx] * BK[3-by-2dy-cy][3-bx-2dx-cx]
 *   V = spatially flipped W, d = 1 - t, double accumulation -> f32.
 * out: [4*OC][R] (column q = k*OC + o, k = 2*by + bx), rows cf-ordered */
void orc_tsubcf(const float *W, const float *BK, int OC, int IC, float *out) {
    const size_t R = (size_t) IC * 9;
#pragma omp parallel for schedule(static)
    for (int o = 0; o < OC; o++) {
        for (int i = 0; i < IC; i++) {
            const float *pw = W + ((size_t) o * IC + i) * 9;
            float V[3][3];
            for (int a = 0; a < 3; a++)
                for (int b = 0; b < 3; b++) V[a][b] = pw[(2 - a) * 3 + (2 - b)];
            for (int by = 0; by < 2; by++)
                for (int bx = 0; bx < 2; bx++) {
                    const int k = by * 2 + bx;
                    float *dst = out + (size_t) (k * OC + o) * R;
                    for (int ty = 0; ty < 3; ty++)
                        for (int tx = 0; tx < 3; tx++) {
                            const int dy = 1 - ty, dx = 1 - tx;
                            double acc = 0;
                            for (int cy = 0; cy < 3; cy++) {
                                const int ay = 3 - by - 2 * dy - cy;
                                if (ay < 0 || ay > 3) continue;
                                for (int cx = 0; cx < 3; cx++) {
                                    const int ax = 3 - bx - 2 * dx - cx;
                                    if (ax < 0 || ax > 3) continue;
                                    acc += (double) V[cy][cx] * (double) BK[ay * 4 + ax];
                                }
                            }
                            dst[i + (size_t) IC * (tx + 3 * ty)] = (float) acc;
                        }
                }
        }
    }
}

/* ------------------------------------------------------------------ */
/* channels-first im2col (patch :201-307): src CL [IC, IW, IH, nb] ->
 * dst [nb*OH*OW][R], R = IC*9, row r = ic + IC*(kw + 3*kh), 3x3, stride 1,
 * zero pad p.  round16 != 0 rounds values to f16 (f16 dst tensor).      */
void orc_im2col_cf(const float *x, int IC, int IW, int IH, int nb, int pad, int round16,
                   float *dst) {
    const int OW = IW + 2 * pad - 2, OH = IH + 2 * pad - 2;
    const size_t R = (size_t) IC * 9;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t) nb * OH * OW; n++) {
        const int ow = (int) (n % OW), oh = (int) ((n / OW) % OH), b = (int) (n / ((int64_t) OW * OH));
        const float *src = x + (size_t) b * IC * IW * IH;
        float *d = dst + (size_t) n * R;
        for (int kh = 0; kh < 3; kh++)
            for (int kw = 0; kw < 3; kw++) {
                const int iw = ow + kw - pad, ih = oh + kh - pad;
                float *dd = d + (size_t) IC * (kw + 3 * kh);
                if (iw < 0 || iw >= IW || ih < 0 || ih >= IH) {
                    for (int c = 0; c < IC; c++) dd[c] = 0.0f;
                } else {
                    const float *s = src + (size_t) IC * (iw + (size_t) IW * ih);
                    if (round16)
                        for (int c = 0; c < IC; c++) dd[c] = orc_f16_to_f32(orc_f32_to_f16(s[c]));
                    else
                        for (int c = 0; c < IC; c++) dd[c] = s[c];
                }
            }
    }
}

/* ------------------------------------------------------------------ */
/* GGML_OP_BILINEAR_GATHER (patch :314-369): torch grid_sample, bilinear,
 * zeros padding, align_corners=False, over feat [C, W*H] channel-fastest.
 * grid interleaved [2, N] (planar=0) or planar [N, 2] (planar=1);
 * dst [C, N] (sp=0) or [N, C] (sp=1).  Tap order k = 0..3 with
 * cx = x0 + (k&1), cy = y0 + (k>>1); acc starts at 0 and adds w*f.     */
void orc_bilinear_gather(const float *feat, int C, int W, int H, const float *grid, int64_t N,
                         int planar, int sp, float *dst) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++) {
        const float gx = planar ? grid[n] : grid[2 * n + 0];
        const float gy = planar ? grid[N + n] : grid[2 * n + 1];
        const float fx = (gx + 1.0f) * 0.5f * (float) W - 0.5f;
        const float fy = (gy + 1.0f) * 0.5f * (float) H - 0.5f;
        const int64_t x0 = (int64_t) floorf(fx);
        const int64_t y0 = (int64_t) floorf(fy);
        const float wx = fx - (float) x0;
        const float wy = fy - (float) y0;
        float *d = dst + (sp ? n : (int64_t) C * n);
        const int64_t ds = sp ? N : 1;
        for (int64_t c = 0; c < C; c++) d[c * ds] = 0.0f;
        for (int k = 0; k < 4; k++) {
            const int64_t cx = x0 + (k & 1);
            const int64_t cy = y0 + (k >> 1);
            if (cx < 0 || cx >= W || cy < 0 || cy >= H) continue;
            const float wgt = ((k & 1) ? wx : 1.0f - wx) * ((k >> 1) ? wy : 1.0f - wy);
            const float *f = feat + (int64_t) C * (cy * W + cx);
            for (int64_t c = 0; c < C; c++) d[c * ds] += wgt * f[c];
        }
    }
}

/* the integer tap selection + f32 weights of the same gather, per point:
 * x0, y0 (int32) and wx, wy (f32) */
void orc_gather_taps(int W, int H, const float *grid, int64_t N, int planar, int32_t *x0o,
                     int32_t *y0o, float *wxo, float *wyo) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++) {
        const float gx = planar ? grid[n] : grid[2 * n + 0];
        const float gy = planar ? grid[N + n] : grid[2 * n + 1];
        const float fx = (gx + 1.0f) * 0.5f * (float) W - 0.5f;
        const float fy = (gy + 1.0f) * 0.5f * (float) H - 0.5f;
        const float fxf = floorf(fx), fyf = floorf(fy);
        x0o[n] = (int32_t) fxf;
        y0o[n] = (int32_t) fyf;
        wxo[n] = fx - (float) (int64_t) fxf;
        wyo[n] = fy - (float) (int64_t) fyf;
    }
}

/* GGML_OP_BIAS_LRELU (patch :372-430): y = leaky(x + b[c], slope), c from
 * axis 0 (CL: i % C) or axis 2 (SP: (i / d01) % C) */
void orc_bias_lrelu(const float *x, const float *b, int64_t n, int C, int64_t d01, int axis,
                    float slope, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const int c = axis == 0 ? (int) (i % C) : (int) ((i / d01) % C);
        const float v = x[i] + b[c];
        y[i] = v > 0.0f ? v : slope * v;
    }
}

/* GGML_OP_SUBPIX_LRELU (patch :432-482): g0/g1 SP [W, H, 2*OC] (row parity
 * by = 0/1, channel q = bx*OC + o) -> dst SP [2W, 2H, OC]:
 *   dst[2n+bx, 2m+by, o] = leaky(g_by[n, m, o + OC*bx] + b[o]) */
void orc_subpix_lrelu(const float *g0, const float *g1, const float *b, int W, int H, int OC,
                      float slope, float *y) {
    const int64_t W2 = 2 * (int64_t) W, H2 = 2 * (int64_t) H;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t) OC * H2; r++) {
        const int64_t yy = r % H2, o = r / H2;
        const float *g = (yy & 1) ? g1 : g0;
        const int64_t ry = yy >> 1;
        const float *se = g + W * (ry + H * o);
        const float *so = g + W * (ry + H * (o + OC));
        float *out = y + r * W2;
        for (int64_t nn = 0; nn < W; nn++) {
            const float v0 = se[nn] + b[o];
            const float v1 = so[nn] + b[o];
            out[2 * nn] = v0 > 0.0f ? v0 : slope * v0;
            out[2 * nn + 1] = v1 > 0.0f ? v1 : slope * v1;
        }
    }
}

/* GGML_OP_SUBPIX_LRELU_CL (patch :485-530): y4 CL [4*OC, W*H, nb] with
 * column q = k*OC + o, k = 2*by + bx -> dst CL [OC, 4*W*H, nb]:
 *   dst[o, (2n+bx) + 2W*(2m+by), b] = leaky(y4[o + OC*k, n + W*m, b] + bias[o]) */
void orc_subpix_lrelu_cl(const float *y4, const float *bias, int OC, int W, int H, int nb,
                         float slope, float *y) {
    const int64_t N = (int64_t) W * H, W2 = 2 * (int64_t) W;
    const int64_t npix = 4 * N * nb;
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < npix; p++) {
        const int64_t nn = p % (4 * N), bb = p / (4 * N);
        const int64_t X = nn % W2, Y = nn / W2;
        const int64_t k = (Y & 1) * 2 + (X & 1);
        const float *src = y4 + OC * k + 4 * (int64_t) OC * ((X >> 1) + W * (Y >> 1) + N * bb);
        float *out = y + (int64_t) OC * p;
        for (int o = 0; o < OC; o++) {
            const float v = src[o] + bias[o];
            out[o] = v > 0.0f ? v : slope * v;
        }
    }
}

/* GGML_OP_UPFIRDN2X (patch :532-572): upfirdn2d(up=2, pad=(2,1)) with a 4x4
 * kernel k4[i + 4*j] over SP [W, H, CB] -> [2W, 2H, CB]:
 *   dst[X, Y] = sum_{i,j} zstuff(src)[X+i-2, Y+j-2] * k4[i + 4j]          */
void orc_upfirdn2x(const float *x, const float *k4, int W, int H, int64_t CB, float *y) {
    const int64_t n_tot = 4 * (int64_t) W * H * CB;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_tot; i++) {
        const int64_t X = i % (2 * W);
        const int64_t Y = (i / (2 * W)) % (2 * H);
        const int64_t cb = i / (4 * (int64_t) W * H);
        const float *xp = x + (int64_t) W * H * cb;
        float acc = 0.0f;
        for (int j = 0; j < 4; j++) {
            const int64_t vy = Y + j - 2;
            if (vy < 0 || vy >= 2 * H || (vy & 1)) continue;
            for (int ii = 0; ii < 4; ii++) {
                const int64_t vx = X + ii - 2;
                if (vx < 0 || vx >= 2 * W || (vx & 1)) continue;
                acc += xp[(vx >> 1) + W * (vy >> 1)] * k4[ii + 4 * j];
            }
        }
        y[i] = acc;
    }
}

/* GGML_OP_CLSP_MUL / GGML_OP_CLSP_LERP (patch :575-626): cl [C, N], m [N]
 *   mul:  dst[n + N*c] = cl[c + C*n] * m[n]
 *   lerp: dst[n + N*c] = cl[c + C*n] * m[n] + o[n + N*c] * (1 - m[n])     */
void orc_clsp(const float *cl, const float *m, const float *o, int C, int64_t N, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t) C * N; i++) {
        const int64_t n = i % N, c = i / N;
        float v = cl[c + (int64_t) C * n] * m[n];
        if (o) v = v + o[i] * (1.0f - m[n]);
        y[i] = v;
    }
}

/* GGML_OP_FLOW_GRID (patch :629-657): fl SP [W, H, 3], xs [N, 2] planar
 * -> dst [N, 3] planar: tanh(fl0)+xs0, tanh(fl1)+xs1, 1/(1+exp(-fl2))     */
void orc_flow_grid(const float *fl, const float *xs, int64_t N, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < 3 * N; i++) {
        const int64_t pln = i / N, n = i % N;
        float v;
        if (pln == 2)
            v = 1.0f / (1.0f + expf(-fl[2 * N + n]));
        else
            v = tanhf(fl[pln * N + n]) + xs[pln * N + n];
        y[i] = v;
    }
}

/* elementwise tanh / sigmoid as ggml's CPU unary ops compute them */
void orc_tanh(const float *x, int64_t n, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = tanhf(x[i]);
}
void orc_sigmoid(const float *x, int64_t n, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------------------ */
/* direct 2-D cross-correlation (ggml_conv_2d_direct semantics, stride 1,
 * dilation 1) on SP maps: x [IC][IH][IW], w [OC][IC][KH][KW] (torch order)
 * -> y [OC][OH][OW], OH = IH + 2p - KH + 1.  f32 accumulation in order
 * (ic, kh, kw) per output element.                                       */
void orc_conv2d_direct(const float *x, int IC, int IH, int IW, const float *w, int OC, int KH,
                       int KW, int pad, float *y) {
    const int OH = IH + 2 * pad - KH + 1, OW = IW + 2 * pad - KW + 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < (int64_t) OC * OH; t++) {
        const int o = (int) (t / OH), oy = (int) (t % OH);
        float *yr = y + ((size_t) o * OH + oy) * OW;
        for (int ox = 0; ox < OW; ox++) yr[ox] = 0.0f;
        for (int i = 0; i < IC; i++) {
            const float *xp = x + (size_t) i * IH * IW;
            const float *wp = w + ((size_t) o * IC + i) * KH * KW;
            for (int kh = 0; kh < KH; kh++) {
                const int iy = oy + kh - pad;
                if (iy < 0 || iy >= IH) continue;
                const float *xr = xp + (size_t) iy * IW;
                for (int kw = 0; kw < KW; kw++) {
                    const float wv = wp[kh * KW + kw];
                    int lo = pad - kw, hi = IW + pad - kw;  /* ox range with valid ix */
                    if (lo < 0) lo = 0;
                    if (hi > OW) hi = OW;
                    for (int ox = lo; ox < hi; ox++) yr[ox] += wv * xr[ox + kw - pad];
                }
            }
        }
    }
}

/* direct 2-D cross-correlation with stride s (dilation 1) on SP maps:
 * x [IC][IH][IW], w [OC][IC][KH][KW] -> y [OC][OH][OW], OH = (IH + 2p - KH) / s + 1.
 * The encoder's strided convs (src/motion_enc.cpp:89-96 via conv2d,
 * src/ops_common.h:12-25).  f32 accumulation in order (ic, kh, kw).      */
void orc_conv2d_s(const float *x, int IC, int IH, int IW, const float *w, int OC, int KH, int KW,
                  int stride, int pad, float *y) {
    const int OH = (IH + 2 * pad - KH) / stride + 1, OW = (IW + 2 * pad - KW) / stride + 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < (int64_t) OC * OH; t++) {
        const int o = (int) (t / OH), oy = (int) (t % OH);
        float *yr = y + ((size_t) o * OH + oy) * OW;
        for (int ox = 0; ox < OW; ox++) yr[ox] = 0.0f;
        for (int i = 0; i < IC; i++) {
            const float *xp = x + (size_t) i * IH * IW;
            const float *wp = w + ((size_t) o * IC + i) * KH * KW;
            for (int kh = 0; kh < KH; kh++) {
                const int iy = oy * stride + kh - pad;
                if (iy < 0 || iy >= IH) continue;
                const float *xr = xp + (size_t) iy * IW;
                for (int kw = 0; kw < KW; kw++) {
                    const float wv = wp[kh * KW + kw];
                    for (int ox = 0; ox < OW; ox++) {
                        const int ix = ox * stride + kw - pad;
                        if (ix >= 0 && ix < IW) yr[ox] += wv * xr[ix];
                    }
                }
            }
        }
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void) n;
#endif
}
