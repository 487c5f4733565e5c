/* tpmd.h — C ABI of the MI355X (gfx950) motion decoder of talking-portrait.cpp.
 *
 * This library replaces the per-frame LIA/StyleGAN motion decoder of the
 * reference (`tp::motion_dec`, src/motion_dec.h:10-49, src/motion_dec.cpp)
 * with hand-written HIP kernels.  Everything above the decoder (tp.h,
 * pipeline, encoders) is unchanged: the reference's motion_dec methods map
 * one-to-one onto the entry points below (see the citations), and the C++
 * shim in talking-portrait.cpp_amd/host/motion_dec.h keeps their exact
 * names and signatures.
 *
 * Conventions (the reference's tp.h contract, include/tp.h:3-10): opaque
 * handle, caller-owned flat buffers, fixed-width types, no exceptions cross
 * this boundary.  Functions returning int return 0 on success and -1 on
 * failure; the reason is then available from tpmd_last_error(ctx).  Every
 * destroy is NULL-safe.  A context is used by one thread at a time.
 *
 * Layouts (ggml "ne" order in the reference, fastest first):
 *   style / latent : [frame][512] f32
 *   image          : [frame][3][R][R] f32, CHW (the reference's img chunks)
 *   feats j        : [r_j*r_j][OC_j] f32, pixel-major channel-fastest
 *                    (menc_result.feats, src/motion_enc.h:12-19)
 *   CL map         : [frame][y][x][channel]  (the fast graph's [C, N, B])
 *   SP map         : [frame][channel][y][x]  (the spatial [W, H, C, B])
 */
#ifndef TPMD_H
#define TPMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TPMD_ABI_VERSION 1
#define TPMD_MAX_STAGES 7
#define TPMD_STYLE_DIM 512

typedef struct tpmd_ctx tpmd_ctx;

/* tp_abi_version (include/tp.h:27) — the decoder library's own ABI level. */
int tpmd_abi_version(void);

/* Create a decoder on HIP device `device`.
 * Replaces backend_t::init + motion_dec construction (src/backend.cpp:9-57,
 * src/tp.cpp:13-41).  ftype "f32" | "f16" follows tp_load's ftype
 * (include/tp.h:33-35, src/tp.cpp:17-30): f16 keeps the big file-f16
 * weights in f16 (f16-in / f32-accumulate MFMA), f32 computes in f32.
 * n_stages: 1..7 pyramid stages (7 = full 512x512 decoder; fewer truncates
 * like TP_MDEC_STAGES, src/motion_dec.cpp:787-792).  stage_ic / stage_oc:
 * NULL for the reference channels {512,512,512,512,256,128,64} /
 * {512,512,512,256,128,64,32} (src/motion_dec.cpp:12-13), or per-stage lists
 * (multiples of 32, stage_ic[j+1] == stage_oc[j]) for reduced test models.
 * Returns NULL on failure (message on stderr). */
tpmd_ctx *tpmd_create(int device, const char *ftype, int n_stages, const int *stage_ic,
                      const int *stage_oc);
void tpmd_destroy(tpmd_ctx *ctx);
/* tp_last_error (include/tp.h:38) */
const char *tpmd_last_error(const tpmd_ctx *ctx);

/* weight flags */
#define TPMD_W_F16_FILE 1 /* tensor is stored f16 in the GGUF (gtype 1) */
#define TPMD_W_FOLDED 2   /* data already carries motion_ae_scale folding */

/* Hand one decoder tensor to the library, by its GGUF name and torch layout
 * (e.g. "dec.convs.3.conv.weight", [1,OC,IC,3,3] row-major), as f32 host
 * data.  Replaces weights_t::load for the dec.* tensors
 * (src/gguf_load.cpp:146-194): unless TPMD_W_FOLDED, the load-time scale
 * folding of motion_ae_scale (src/motion_enc.cpp:14-45) is applied here;
 * with ftype f16, tensors flagged TPMD_W_F16_FILE with >= 4096 elements are
 * stored f16 (src/gguf_load.cpp:149-153).  n = element count (checked). */
int tpmd_set_weight(tpmd_ctx *ctx, const char *name, const float *data, int64_t n, int flags);

/* The decoder tensors this context expects, i = 0, 1, ...: GGUF name,
 * element count and whether the tensor is a 2-D-or-larger weight (stored
 * f16 in an f16 GGUF).  Returns the name, or NULL past the last tensor.
 * Replaces the weight list the reference walks implicitly through
 * weights_t lookups (src/motion_dec.cpp:249-261) and motion_dec_host_tensors
 * (src/motion_dec.cpp:17-29). */
const char *tpmd_weight_name(const tpmd_ctx *ctx, int i, int64_t *n, int *is_matrix);

/* Hand every decoder tensor of a motion_ae GGUF v3 checkpoint
 * (motion_ae_{f32,f16}.gguf, general.architecture "float-motion-ae") to the
 * context, as tpmd_set_weight does: replaces weights_t::load for the dec.*
 * tensors (src/gguf_load.cpp:51-197, src/tp.cpp:33-35).  Tensors the file
 * lacks are reported by tpmd_prepare ("missing tensor <name>").  Returns 0,
 * or -1 with the reason (file defects as the reference words them: "not a
 * GGUF file", "unsupported GGUF version", "unexpected architecture", "tensor
 * <name> out of bounds", ...) in err[0..err_size). */
int tpmd_load_gguf(tpmd_ctx *ctx, const char *path, char *err, size_t err_size);
/* One tensor of a GGUF v3 file as f32 (F16 tensors widened exactly);
 * *is_f16 = stored as F16.  out may be NULL to query the element count.
 * Returns the element count, or -1 with the reason in err.  Needs no
 * device. */
int64_t tpmd_gguf_read_tensor(const char *path, const char *name, float *out, int64_t cap,
                              int *is_f16, char *err, size_t err_size);

/* motion_dec::prepare (src/motion_dec.h:38, src/motion_dec.cpp:31-226):
 * S_aug demodulation Gram rows, composed sub-pixel up-conv kernels, cf GEMM
 * matrices; uploads every derived tensor.  Fails naming the first missing
 * tensor ("missing tensor <name>"). */
int tpmd_prepare(tpmd_ctx *ctx);

/* motion_dec::build (src/motion_dec.h:41, src/motion_dec.cpp:659-1135):
 * allocate the persistent per-batch buffers for up to max_batch frames per
 * call (1..256) and the stage constants.  Requires tpmd_prepare. */
int tpmd_build(tpmd_ctx *ctx, int max_batch);
/* frames per call chosen at build (motion_dec::batch, src/motion_dec.h:28) */
int tpmd_batch(const tpmd_ctx *ctx);
/* output resolution R = 8 << (n_stages - 1) */
int tpmd_out_res(const tpmd_ctx *ctx);

/* motion_dec::set_feats (src/motion_dec.h:43, src/motion_dec.cpp:1137-1160):
 * feats[j] = [r_j*r_j][OC_j] f32 host, j < n_stages; stored f16 in f16
 * mode.  Requires tpmd_build ("decoder not built"). */
int tpmd_set_feats(tpmd_ctx *ctx, const float *const *feats);
/* same from device memory (f32) */
int tpmd_set_feats_device(tpmd_ctx *ctx, const float *const *feats_dev);

/* motion_dec::decode_batch (src/motion_dec.h:46-47,
 * src/motion_dec.cpp:1190-1220): n (1..batch) latents -> n frames.
 * styles: [n][512]; imgs: [n][3][R][R]; both host pointers
 * (on_device = 0, synchronous like the reference) or device pointers
 * (on_device = 1, asynchronous).
 *
 * Device-resident calls on a caller's stream (tpmd_set_stream) are
 * enqueued on that stream in call order.  On the decoder's own stream (the
 * default) consecutive calls rotate over three lanes, each with its own
 * buffers and stream, so their launch chains overlap on the GPU:
 *   - a call reads `styles` after all work enqueued before it on HIP's null
 *     stream (e.g. torch's default stream), and null-stream work enqueued
 *     after the call runs after that read, so the caller may refill the
 *     latent buffer on the null stream right away;
 *   - a call whose `imgs` overlaps the frame buffer of an earlier call still
 *     in flight writes its frames after that call's, so one frame buffer
 *     may be reused: after tpmd_sync it holds the last call's frames;
 *   - frames are complete only after tpmd_sync (latents written on another
 *     stream need that stream synchronised first, or tpmd_set_stream). */
int tpmd_decode_batch(tpmd_ctx *ctx, const float *styles, int n, float *imgs, int on_device);

/* Taps of the decode chain: device copies of the buffers that the batched
 * decoder passes between its launches, for per-stage parity checks of the
 * kernels exactly as decode_batch runs them.  The reference's tap plan
 * (motion_dec::build(be, with_taps), src/motion_dec.cpp:805-883, dumped by
 * tools/tp-parity.cpp:252-282) names its taps conv1_4, r<r>.conv1,
 * r<r>.conv2, r<r>.flowmap, r<r>.out, r<r>.rgb; here they are the fast
 * chain's own buffers, in its layouts (stage j: r = 8 << j, C = OC_j; the
 * activation type is f16 in f16 mode, else f32):
 *   TPMD_TAP_TRUNK  stage -1 (conv1 output, r = 4, C = IC_0) and
 *                   j < n_stages - 1 (trunk, r<r>.out): CL [n][r][r][C]
 *                   activation type, multiplied by the style of the
 *                   up-conv that reads it;
 *   TPMD_TAP_C1     up-conv output (r<r>.conv1): CL [n][r][r][C]
 *                   activation type, multiplied by the dense conv's style;
 *   TPMD_TAP_OUT    dense-conv output (r<r>.conv2): CL [n][r][r][C] f32,
 *                   only for stages whose tail runs in a kernel of its own;
 *   TPMD_TAP_FLOW   flow map with skip (r<r>.flowmap): SP [n][3][r][r] f32
 *                   (the last stage stores it only while tapped);
 *   TPMD_TAP_RGB    rgb with skip (r<r>.rgb): SP [n][3][r][r] f32, stages
 *                   j < n_stages - 1 (the last one is the frame).
 * tpmd_set_tap registers (dst a device buffer of `bytes`) or removes (dst
 * NULL) one tap; every later decode_batch copies frames [0, n) of that
 * buffer into it on the decoder's stream (a decode with taps set runs on
 * one lane), failing if `bytes` is too small.  tpmd_tap_frame_bytes gives
 * the bytes per frame, or -1 where the chain holds no such buffer. */
/* The reference's tap plan for one frame (motion_dec::decode with a
 * tap_sink after build(be, true), src/motion_dec.cpp:794-888 and
 * :1162-1188; dumped by tools/tp-parity.cpp:252-282): the style [512]
 * (host) is decoded through the per-stage entry points' f32 kernels (styled
 * convs with f32 output, the standalone stage tail storing trunk and warp),
 * and every tap is handed to cb as host f32 in the reference's names and
 * torch layouts, in decode order: conv1_4 [1,C0,4,4]; then per stage
 * r = 8 << j: r<r>.conv1, r<r>.conv2 [1,OC,r,r]; r<r>.flowmap [1,3,r,r];
 * r<r>.grid [1,r,r,2]; r<r>.warp, r<r>.out [1,OC,r,r]; r<r>.rgb [1,3,r,r].
 * data is valid during the call; a nonzero return stops with -1.  img
 * (host [3][R][R], or NULL) receives the frame.  Synchronous. */
typedef int (*tpmd_tap_cb)(const char *name, const float *data, int ndim, const int64_t *shape, void *ud);
int tpmd_decode_taps(tpmd_ctx *ctx, const float *style, float *img, tpmd_tap_cb cb, void *ud);

#define TPMD_TAP_TRUNK 0
#define TPMD_TAP_C1 1
#define TPMD_TAP_OUT 2
#define TPMD_TAP_FLOW 3
#define TPMD_TAP_RGB 4
#define TPMD_TAP_KINDS 5
int tpmd_set_tap(tpmd_ctx *ctx, int kind, int stage, void *dst, int64_t bytes);
int64_t tpmd_tap_frame_bytes(const tpmd_ctx *ctx, int kind, int stage);
/* Frame output path of a clip (the generation loop's decode stage,
 * src/pipeline.cpp:160-185): n_frames latents (host [n][512]) are decoded
 * in launches of `batch` frames (rotating over the decoder's lanes when it
 * runs on its own stream); while launch k runs, the frames of launch k-1
 * come back over a copy stream into pinned staging and are handed over.  format TPMD_FRAME_F32: [3][R][R] f32 per frame, as decode_batch;
 * TPMD_FRAME_RGB24: [R][R][3] u8 per frame, converted on the GPU with the
 * video writer's rule (tools/tp-cli.cpp:43-53: clamp to [-1,1],
 * (v+1)/2*255, truncate), a quarter of the bytes.  out: host buffer for all
 * frames, or NULL (pinned memory, e.g. from hipHostMalloc, takes the
 * downloads directly; pageable memory is filled from pinned staging by
 * helper threads); cb: called per frame in order with the frame (valid only
 * during the call, tp_frame_cb semantics, include/tp.h:57-62), or NULL;
 * a nonzero return stops decoding.  Returns n_frames (also when stopped, as
 * generate_impl does) or -1.  The first call allocates one slot of device
 * and one of pinned host memory per lane (three) for `batch` frames, kept
 * by the context. */
#define TPMD_FRAME_F32 0
#define TPMD_FRAME_RGB24 1
typedef int (*tpmd_frame_cb)(int64_t frame_idx, const void *frame, void *ud);
int64_t tpmd_decode_frames(tpmd_ctx *ctx, const float *styles, int64_t n_frames, int format, void *out,
                           tpmd_frame_cb cb, void *ud);

/* motion_dec::decode (src/motion_dec.h:44-45, :1162-1188): one frame. */
int tpmd_decode(tpmd_ctx *ctx, const float *style, float *img);
/* wait for work enqueued by on_device calls */
int tpmd_sync(tpmd_ctx *ctx);
/* enqueue all further work of this context on `stream` (a hipStream_t of
 * the context's device, e.g. the caller's framework stream; NULL = HIP's
 * null stream), after the work in flight on the context's streams and on
 * the previous caller stream has finished.  A new context uses a
 * non-blocking stream of its own.  No
 * reference counterpart: ggml owns its stream (src/backend.cpp:169-177);
 * callers that share device buffers with other stream users need this
 * ordering. */
int tpmd_set_stream(tpmd_ctx *ctx, void *stream);
/* Whether decode_batch / decode_frames replay each lane's launch chain as a
 * HIP graph (captured on the first call for a frame count and frame buffer,
 * up to 4 per lane kept) instead of enqueuing its launches one by one;
 * frames are the same bits either way.  On by default; TPMD_GRAPHS=0 in the
 * environment at tpmd_create turns it off.  Waits for work in flight.  No
 * entry point of the reference: there ggml-cuda's build option
 * GGML_CUDA_GRAPHS decides whether a graph's launches are captured as a
 * CUDA graph (off in its cuda preset, CMakePresets.json:24-33; its
 * steady-state allocation check expects capture, bench/tp-allocproof.cpp:
 * 103-107). */
int tpmd_set_graphs(tpmd_ctx *ctx, int enable);

/* Per-stage timing of the next decode_batch: when enabled, the call records
 * HIP events around each launch group and stores microseconds into
 * us[0..n_slots) (slot 0 = style + demod + conv1, then 3 per stage: up-conv,
 * dense conv, tail; stages with OC <= 128 run the tail inside the dense conv,
 * so their dense slot holds both and their tail slot is empty).  Returns the
 * slot count, or -1. */
int tpmd_profile_stages(tpmd_ctx *ctx, int enable);
int tpmd_stage_times(const tpmd_ctx *ctx, float *us, int max_slots);

/* Sustained f16 MFMA rate of this GPU (no counterpart in the reference: the
 * benchmark's roofline reads it beside the published peak).  Every SIMD
 * runs four waves of independent v_mfma_f32_32x32x16_f16 on all-zero
 * (random_operands = 0) or pseudo-random f16 operands in [-1, 1) for `iters`
 * iterations of 8 MFMAs; *tflops gets the rate over 10 timed launches and
 * *core_ghz the core clock one wave saw.  The MI355X lowers its clock under
 * such a load by an amount that depends on the operand bits, so the random
 * figure is the ceiling of an MFMA-bound kernel.  Synchronous on the null
 * stream; allocates and frees a small device buffer.  Returns 0 or -1. */
int tpmd_probe_mfma_f16(int random_operands, int iters, float *tflops, float *core_ghz);

/* ---- per-stage entry points on DEVICE buffers (f32 in / f32 out) -------
 * These run one piece of the decoder with the context's weights, for
 * parity tests and per-stage measurement.  `stream` is a hipStream_t
 * (NULL = HIP's null stream); they are asynchronous on it. */

/* ModulatedConv2d with demodulation + FusedLeakyReLU (styled_conv /
 * styled_conv_up / styled_conv_input, src/motion_dec.cpp:357-433):
 * conv = 0 for dec.conv1, 1 + i for dec.convs.i (even i: 2x sub-pixel
 * up-conv).  x: CL [n][H][W][IC]; s: [n][IC] style of this conv (the
 * demodulation is computed from it); y: CL [n][H'][W'][OC]. */
int tpmd_modconv(tpmd_ctx *ctx, int conv, const float *x, int n, int H, int W, const float *s,
                 float *y, void *stream);

/* tpmd_modconv for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, kernels
 * and results as tpmd_modconv, but its scratch (the style-multiplied
 * input, 1/den, split-K partial sums; each rounded up to 256 bytes) lives
 * in a static device array of TPMD_STATIC_SCRATCH_BYTES per GPU, resolved
 * when a context is created on that GPU and held until the process ends;
 * the call allocates nothing.  A call whose scratch exceeds it fails
 * ("needs N bytes of scratch").  All calls on one GPU share the array, from
 * every context: calls that overlap on one GPU (different streams, or
 * contexts used from several threads) race. */
#define TPMD_STATIC_SCRATCH_BYTES ((size_t) 16 << 20)
int tpmd_modconv_static(tpmd_ctx *ctx, int conv, const float *x, int n, int H, int W, const float *s,
                        float *y, void *stream);

/* Stage tail of stage j (src/motion_dec.cpp:1077-1108): ToFlow (+ flow
 * skip), flow head, grid_sample warp of feats j, warp/trunk blend, ToRGB
 * (+ rgb skip).  out: CL [n][r][r][C] dense-conv output; s_flow: [n][C];
 * flow_prev / rgb_prev: SP [n][3][r/2][r/2] or NULL (stage 0); outputs
 * flow: SP [n][3][r][r] (or NULL), trunk: CL f32 (or NULL), rgb: SP,
 * warp: CL f32 (or NULL). */
int tpmd_stage_tail(tpmd_ctx *ctx, int j, const float *out, int n, const float *s_flow,
                    const float *flow_prev, const float *rgb_prev, float *flow, float *trunk,
                    float *rgb, float *warp, void *stream);

/* Dense conv of stage j followed by the stage tail, exactly as decode runs
 * them (fused into one kernel when OC_j <= 128, src/motion_dec.cpp:357-373
 * then :1077-1108): c1: CL [n][r][r][OC_j] f32 up-conv output (before this
 * conv's modulation); s_conv: [n][OC_j] this conv's style (demodulation
 * computed from it); other arguments as tpmd_stage_tail, trunk CL f32. */
int tpmd_stage_conv_tail(tpmd_ctx *ctx, int j, const float *c1, int n, const float *s_conv,
                         const float *s_flow, const float *flow_prev, const float *rgb_prev,
                         float *flow, float *trunk, float *rgb, float *warp, void *stream);

/* ---- motion encoder ---------------------------------------------------- */

/* tp::motion_enc (src/motion_enc.h:20-30, src/motion_enc.cpp:50-184): the
 * LIA EncoderApp pyramid (EqualConv2d / FusedLeakyReLU / Blur ResBlocks,
 * 512 -> 4), the 5-layer EqualLinear fc chain and the baked Direction Q.
 * It runs once per portrait; its feats feed tpmd_set_feats_device. */
typedef struct tpme_ctx tpme_ctx;

/* device / ftype as tpmd_create (ftype "f16": tensors kept f16 are GEMM
 * operands in f16, with the other operand rounded to f16, as ggml's
 * im2col and vec_dot convert them).  n_blocks: 7 for the 512x512 encoder;
 * ch_in / ch_out: NULL for the reference widths {32,64,128,256,512,512,512}
 * / {64,128,256,512,512,512,512} (src/motion_enc.cpp:47-48), or per-ResBlock
 * lists (multiples of 32, ch_in[i+1] == ch_out[i]) for reduced test models.
 * The input image is (4 << n_blocks) pixels square.  NULL on failure. */
tpme_ctx *tpme_create(int device, const char *ftype, int n_blocks, const int *ch_in, const int *ch_out);
void tpme_destroy(tpme_ctx *ctx);
const char *tpme_last_error(const tpme_ctx *ctx);
/* the encoder tensors in GGUF names (enc.* and dec.direction.Q), i = 0.. ;
 * NULL past the end */
const char *tpme_weight_name(const tpme_ctx *ctx, int i, int64_t *n, int *is_matrix);
/* as tpmd_set_weight: raw values in torch order, motion_ae_scale folded at
 * load unless TPMD_W_FOLDED (src/motion_enc.cpp:14-45) */
int tpme_set_weight(tpme_ctx *ctx, const char *name, const float *data, int64_t n, int flags);
/* weights_t::load for the encoder's tensors (src/gguf_load.cpp:51-197), as
 * tpmd_load_gguf: every enc.* tensor and dec.direction.Q of a
 * "float-motion-ae" GGUF v3 file through tpme_set_weight (F16 tensors with
 * TPMD_W_F16_FILE); 0, or -1 with the reason in err[0..err_size) */
int tpme_load_gguf(tpme_ctx *ctx, const char *path, char *err, size_t err_size);
/* conv weights to tap-major GEMM operands, device upload; "missing tensor
 * <name>" when one was not set */
int tpme_prepare(tpme_ctx *ctx);
/* motion_enc::run (src/motion_enc.cpp:50-184): image [3][R][R] f32 CHW in
 * [-1,1] (host, or device when on_device != 0).  Synchronous. */
int tpme_run(tpme_ctx *ctx, const float *image, int on_device);
/* the last run's menc_result vectors (src/motion_enc.h:10-18), host copies:
 * appearance [512], lambda [20], motion [512] = Q lambda; any may be NULL */
int tpme_result(const tpme_ctx *ctx, float *appearance, float *lambda, float *motion);
/* feats j of the last run: device [r*r][C] f32, r = 8 << j (= encoder level
 * n_blocks - 1 - j), valid until the next run or destroy; pass all seven
 * to tpmd_set_feats_device.  NULL on a bad index or before a run. */
const float *tpme_feat(const tpme_ctx *ctx, int j, int *C, int *r);
/* host copy of pyramid level l (menc.conv<l>, l = 0..n_blocks), CL
 * [r*r][C] f32; returns the element count, or -1 (dst NULL: count only) */
int64_t tpme_level(tpme_ctx *ctx, int level, float *dst);

/* ---- flow-matching transformer ------------------------------------------ */

/* tp::fmt_model (src/fmt.h:9-36, src/fmt.cpp): 8 DiT blocks with per-frame
 * adaLN modulation and a banded attention mask, CFG-batched over the three
 * condition branches [uncond, full, audio_only]; and its ODE chunk sampler
 * (sample_chunk, src/pipeline.cpp:12-91). */
typedef struct tpfm_ctx tpfm_ctx;
/* fmt_model's hyper-parameters; defaults as src/fmt.h:10-16 */
typedef struct tpfm_config {
    int dim_h, depth, n_heads, dim_w, dim_a, dim_e;
    int chunk_frames, prev_frames, attn_window, t_freq_dim, nfe;
    float mlp_ratio, ln_eps, a_cfg, e_cfg, r_cfg;
} tpfm_config;
void tpfm_default_config(tpfm_config *cfg);
/* the float.fmt.* keys of a "float-fmt" GGUF file (src/fmt.cpp:8-26) over
 * the defaults; 0, or -1 with the reason in err */
int tpfm_read_config(const char *gguf_path, tpfm_config *cfg, char *err, size_t err_size);
/* ftype as tpmd_create.  Constraints of this build: dim_h % n_heads == 0,
 * head dim <= 256, attn_window <= 7, and dim_h, dim_w, t_freq_dim and the
 * MLP width multiples of 32.  NULL on failure (message on stderr). */
tpfm_ctx *tpfm_create(int device, const char *ftype, const tpfm_config *cfg);
void tpfm_destroy(tpfm_ctx *ctx);
const char *tpfm_last_error(const tpfm_ctx *ctx);
/* the FMT tensors (GGUF names), i = 0.. ; NULL past the end */
const char *tpfm_weight_name(const tpfm_ctx *ctx, int i, int64_t *n, int *is_matrix);
/* values as stored (no load-time folds for the FMT); TPMD_W_F16_FILE as
 * tpmd_set_weight (the f16 keep rule of src/gguf_load.cpp:149-153) */
int tpfm_set_weight(tpfm_ctx *ctx, const char *name, const float *data, int64_t n, int flags);
/* every FMT tensor of a "float-fmt" GGUF v3 file; 0 or -1 with err */
int tpfm_load_gguf(tpfm_ctx *ctx, const char *path, char *err, size_t err_size);
/* device upload; "missing tensor <name>" when one was not set */
int tpfm_prepare(tpfm_ctx *ctx);
/* fmt_model::forward (src/fmt.h:27-31): x60 [total][dim_w], cond
 * [3][total][dim_w+dim_a+dim_e], flow time t -> v_out [3][total][dim_w];
 * host buffers, synchronous */
int tpfm_forward(tpfm_ctx *ctx, const float *x60, const float *cond, float t, float *v_out);
/* sample_chunk (src/pipeline.cpp:12-91): the CFG condition rows from wr
 * [dim_w], prev_wa [prev][dim_a], cond_audio [chunk][dim_a] and emotion
 * (-1: none), then nfe - 1 Euler steps of the CFG-combined velocity from x0
 * [chunk][dim_w] with prev_x [prev][dim_w] -> motion_out [chunk][dim_w];
 * host buffers, synchronous */
int tpfm_sample_chunk(tpfm_ctx *ctx, const float *wr, const float *prev_x, const float *prev_wa,
                      const float *cond_audio, int emotion, const float *x0, float *motion_out);

/* ---- op-level entry points (no context) ------------------------------- */

/* GGML_OP_BILINEAR_GATHER (patches/ggml-tp-ops.patch:41-60, :104-111,
 * CUDA :688-752): torch grid_sample, bilinear, zeros padding,
 * align_corners=False.  feat: [W*H][C] channel-fastest, f32 (feat_f16 = 0)
 * or IEEE f16 (feat_f16 = 1); grid: interleaved [N][2] (planar = 0, the
 * ggml [2, N]) or planar [2][N] (planar = 1, ggml_bilinear_gather_planar);
 * dst: [N][C] (sp = 0) or [C][N] (sp = 1, ggml_bilinear_gather_sp).
 * Device pointers; returns 0 or -1 (invalid arguments). */
int tpmd_gather(const void *feat, int feat_f16, int C, int W, int H, const float *grid, int64_t N,
                int planar, int sp, float *dst, void *stream);
/* the gather's integer tap selection and weights: x0 = floor(fx),
 * y0 = floor(fy), wx = fx - x0, wy = fy - y0 per point (device pointers) */
int tpmd_gather_taps(const float *grid, int W, int H, int64_t N, int planar, int32_t *x0,
                     int32_t *y0, float *wx, float *wy, void *stream);
/* n CHW f32 frames [n][3][R][R] -> [n][R][R][3] u8 with the video writer's
 * conversion (tools/tp-cli.cpp:43-53); device pointers, R*R % 4 == 0 */
int tpmd_frames_to_rgb24(const float *chw, int n, int R, uint8_t *rgb, void *stream);
/* GGML_OP_UPFIRDN2X (patch :128-134, :996-1045): SP [CB][H][W] -> [CB][2H][2W] */
int tpmd_upfirdn2x(const float *x, const float *k4, float *y, int W, int H, int64_t CB,
                   void *stream);
/* GGML_OP_FLOW_GRID (patch :94-102, :1082-1104): fl [3][N], xs [2][N] -> [3][N] */
int tpmd_flow_grid(const float *fl, const float *xs, float *y, int64_t N, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TPMD_H */
