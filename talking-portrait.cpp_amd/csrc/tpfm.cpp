// Flow-matching transformer context behind the tpfm_* C ABI: the reference's
// fmt_model (src/fmt.h:9-36) — weights, prepare, the CFG-batched forward
// (src/fmt.cpp:44-205) — and its chunk sampler (src/pipeline.cpp:12-91), on
// the k_fmt.hip kernels and the MFMA GEMM of k_enc.hip; the f16 linears'
// products on hipBLASLt.  Host code only.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "tpmd_guard.h"
#include "tpmd.h"
#include "tpmd_fmt.h"

using namespace tpmd;

namespace {

std::string ffmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string ffmt(const char *f, ...) {
    char b[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(b, sizeof b, f, ap);
    va_end(ap);
    return b;
}

struct FTensor {
    std::vector<float> data;
    int flags = 0;
};

int round32(int v) { return (v + 31) / 32 * 32; }

// split-K factor of a linear layer over `rows` tokens: about 1024
// workgroups (the GEMM's 64 x 64 tiles are few at 180 rows, and a short k
// loop per workgroup hides the load latency), at least 2 k tiles each, and
// at most 8 splits, whose f32 partials of all rows are written and read back
// (measured on MI355X, a 50-frame chunk: no cap 8.2 ms, at most 8 splits
// 7.6-7.7, at most 4 8.0-8.2, at most 2 10.2-10.3)
int lin_splits(int rows, int out, int in) {
    const int tiles = ((rows + 63) / 64) * ((out + 63) / 64);
    const int T = in / 32;
    return std::max(1, std::min(std::min(1024 / std::max(tiles, 1), T / 2), 8));
}

}  // namespace

struct tpfm_ctx {
    int device = 0;
    bool f16 = false;
    tpfm_config cfg{};
    int T = 60, B = 3, CD = 1031, CDp = 1056, MLP = 4096;
    std::string err;
    hipStream_t stream = nullptr;
    std::vector<std::pair<std::string, std::vector<int64_t>>> tensors;
    std::map<std::string, FTensor> host;
    bool prepared = false;
    std::vector<void *> allocs;

    struct Lin {  // a linear layer as the GEMM's A operand [out][in (padded)]
        void *W = nullptr;
        float *b = nullptr;
        bool f16 = false;
        int out = 0, in = 0;
    };
    Lin cemb, xemb, fin_lin;
    // every adaLN modulation (each block's 6H rows, then the final layer's 2H)
    // reads the same silu(c): one stacked layer, one GEMM per forward
    Lin mods;
    struct Block {
        Lin qkv, proj, fc1, fc2;
    };
    std::vector<Block> blocks;
    float *t0w = nullptr, *t0b = nullptr, *t2w = nullptr, *t2b = nullptr;  // t-embedder (GEMV, f32 values)
    bool t0_16 = false, t2_16 = false;
    float *pos = nullptr;
    std::vector<float> t_freqs;
    std::vector<float> h_cond, h_x60;  // sample_chunk's host staging (sized at prepare)

    // activations
    float *tfk = nullptr, *tf = nullptr, *te0 = nullptr, *te = nullptr;
    float *cond_f = nullptr, *clin = nullptr, *x60 = nullptr, *x1 = nullptr, *x = nullptr;
    float *mod = nullptr, *qkv = nullptr, *v = nullptr;  // mod: [rows][mods.out]
    float *ws = nullptr;  // split-K partials, or a library GEMM's f32 product

    // The f16 linears (f16 weights and operand) run their product on hipBLASLt
    // (f16 operands, f32 accumulation and output into ws) and the epilogue
    // (bias, activation, adaLN gate, residual, operand copy) on the split-K
    // pass of k_enc.hip.  180 token rows against up to 12.6 MB of weights
    // leave the own 64 x 64 tile GEMM latency-bound (one forward's linears
    // about 820 us with their split-K passes); the library's kernels for
    // these shapes sum to about 290 us (measured in one graph on MI355X).
    // A linear with only a bias after the product (qkv, the stacked adaLN
    // layer, the final layer, the embedders) takes the bias in the library's
    // epilogue and writes its f32 output directly (no epilogue pass).  One
    // plan per (rows, out, in, direct), made at prepare; TPFM_BLASLT=0 keeps
    // every linear on the own GEMM.
    struct LtPlan {
        hipblasLtMatmulDesc_t md = nullptr;
        hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
        hipblasLtMatmulAlgo_t algo{};
        size_t ws = 0;
        bool bias = false;  // the library's epilogue adds a bias (direct plans)
    };
    hipblasLtHandle_t lt = nullptr;
    void *lt_ws = nullptr;
    static constexpr size_t LT_WS = (size_t) 32 << 20;
    std::map<std::tuple<int, int, int, bool>, LtPlan> lt_plans;
    void free_lt() {
        for (auto &kv : lt_plans) {
            if (kv.second.md) (void) hipblasLtMatmulDescDestroy(kv.second.md);
            if (kv.second.la) (void) hipblasLtMatrixLayoutDestroy(kv.second.la);
            if (kv.second.lb) (void) hipblasLtMatrixLayoutDestroy(kv.second.lb);
            if (kv.second.ld) (void) hipblasLtMatrixLayoutDestroy(kv.second.ld);
        }
        lt_plans.clear();
        lt_ws = nullptr;  // one of allocs
    }
    void *cond_a = nullptr, *sc_a = nullptr, *x60_a = nullptr, *h_a = nullptr, *o_a = nullptr, *m1_a = nullptr;

    bool hip_ok(hipError_t e, const char *what) {
        if (e == hipSuccess) return true;
        err = ffmt("%s: %s", what, hipGetErrorString(e));
        return false;
    }
    void *dalloc(size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes < 256 ? 256 : bytes) != hipSuccess) {
            err = ffmt("hipMalloc of %zu bytes failed", bytes);
            return nullptr;
        }
        allocs.push_back(p);
        return p;
    }
    template <typename T>
    T *upload(const std::vector<T> &v) {
        T *p = (T *) dalloc(v.size() * sizeof(T));
        if (!p) return nullptr;
        if (!hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "upload")) return nullptr;
        return p;
    }
    const FTensor *need(const std::string &name) {
        auto it = host.find(name);
        if (it == host.end()) {
            if (err.empty()) err = "missing tensor " + name;
            return nullptr;
        }
        return &it->second;
    }
    bool kept16(const FTensor &t) const { return f16 && (t.flags & TPMD_W_F16_FILE) && t.data.size() >= 4096; }
    std::vector<float> dev_value(const FTensor &t) const {
        std::vector<float> v = t.data;
        if (kept16(t))
            for (auto &x : v) x = (float) (_Float16) x;
        return v;
    }
    size_t asz(bool h) const { return h ? 2 : 4; }
    void free_all() {
        free_lt();
        for (void *p : allocs) (void) hipFree(p);
        allocs.clear();
    }
    ~tpfm_ctx() {
        if (device >= 0) (void) hipSetDevice(device);
        free_all();
        if (lt) (void) hipblasLtDestroy(lt);
        if (stream) (void) hipStreamDestroy(stream);
    }
};

namespace {

bool check(tpfm_ctx *c) {
    if (!c) return false;
    c->err.clear();
    if (hipSetDevice(c->device) != hipSuccess) {
        c->err = "hipSetDevice failed";
        return false;
    }
    return true;
}

void make_tensor_list(tpfm_ctx *c) {
    const int64_t H = c->cfg.dim_h, M = c->MLP;
    auto &v = c->tensors;
    auto add = [&](const std::string &n, std::vector<int64_t> s) { v.push_back({n, std::move(s)}); };
    add("t_embedder.mlp.0.weight", {H, c->cfg.t_freq_dim});
    add("t_embedder.mlp.0.bias", {H});
    add("t_embedder.mlp.2.weight", {H, H});
    add("t_embedder.mlp.2.bias", {H});
    add("c_embedder.weight", {H, c->CD});
    add("c_embedder.bias", {H});
    add("x_embedder.proj.weight", {H, c->cfg.dim_w});
    add("x_embedder.proj.bias", {H});
    add("pos_embed", {1, c->T, H});
    for (int i = 0; i < c->cfg.depth; i++) {
        const std::string b = ffmt("blocks.%d", i);
        add(b + ".adaLN_modulation.1.weight", {6 * H, H});
        add(b + ".adaLN_modulation.1.bias", {6 * H});
        add(b + ".attn.qkv.weight", {3 * H, H});
        add(b + ".attn.qkv.bias", {3 * H});
        add(b + ".attn.proj.weight", {H, H});
        add(b + ".attn.proj.bias", {H});
        add(b + ".mlp.fc1.weight", {M, H});
        add(b + ".mlp.fc1.bias", {M});
        add(b + ".mlp.fc2.weight", {H, M});
        add(b + ".mlp.fc2.bias", {H});
    }
    add("decoder.adaLN_modulation.1.weight", {2 * H, H});
    add("decoder.adaLN_modulation.1.bias", {2 * H});
    add("decoder.linear.weight", {c->cfg.dim_w, H});
    add("decoder.linear.bias", {c->cfg.dim_w});
}

// weights [out_j][in] of the layers `bases` (rows stacked in that order) ->
// operand [sum out_j][in_pad] (zero columns past in), f16 when kept f16 (all
// stacked layers must agree), biases stacked alike
bool make_lin_stack(tpfm_ctx *c, tpfm_ctx::Lin &L, const std::vector<std::pair<std::string, int>> &bases, int in,
                    int in_pad) {
    int out = 0;
    for (const auto &bo : bases) out += bo.second;
    L.out = out;
    L.in = in_pad;
    std::vector<float> a((size_t) out * in_pad, 0.0f), bias;
    int o0 = 0;
    for (size_t j = 0; j < bases.size(); j++) {
        const FTensor *w = c->need(bases[j].first + ".weight"), *b = c->need(bases[j].first + ".bias");
        if (!w || !b) return false;
        const bool f16 = c->kept16(*w);
        if (j == 0) L.f16 = f16;
        else if (f16 != L.f16) {
            c->err = "tpfm_prepare: " + bases[0].first + " and " + bases[j].first + " stored with mixed types";
            return false;
        }
        const int oj = bases[j].second;
        const std::vector<float> dv = c->dev_value(*w);
        for (int o = 0; o < oj; o++)
            for (int i = 0; i < in; i++) a[(size_t) (o0 + o) * in_pad + i] = dv[(size_t) o * in + i];
        bias.insert(bias.end(), b->data.begin(), b->data.end());
        o0 += oj;
    }
    if (L.f16) {
        std::vector<_Float16> h(a.size());
        for (size_t i = 0; i < a.size(); i++) h[i] = (_Float16) a[i];
        L.W = c->upload(h);
    } else {
        L.W = c->upload(a);
    }
    L.b = c->upload(bias);
    return L.W && L.b;
}

bool make_lin(tpfm_ctx *c, tpfm_ctx::Lin &L, const std::string &base, int out, int in, int in_pad) {
    return make_lin_stack(c, L, {{base, out}}, in, in_pad);
}

// the hipBLASLt plan of an f16 linear over `rows` token rows, made once:
// D (L.out x rows, column-major: [rows][L.out]) = W^T-stored-as-[L.in x L.out]^T
// x X-stored-as-[L.in x rows], f16 operands, f32 accumulation and output
// (into ws; direct: plus the f32 bias per output feature, into Y).  False
// (and no plan) where the library has no kernel for the shape: that layer
// keeps the own GEMM.
bool lt_plan(tpfm_ctx *c, const tpfm_ctx::Lin &L, int rows, bool direct) {
    const auto key = std::make_tuple(rows, L.out, L.in, direct);
    if (c->lt_plans.count(key)) return true;
    tpfm_ctx::LtPlan P;
    bool ok = hipblasLtMatmulDescCreate(&P.md, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    ok = ok && hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == HIPBLAS_STATUS_SUCCESS;
    P.bias = direct && L.b;
    if (P.bias) {
        const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
        const hipDataType bt = HIP_R_32F;
        const void *bp = L.b;
        ok = ok &&
             hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof ep) ==
                 HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt) ==
                 HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof bp) ==
                 HIPBLAS_STATUS_SUCCESS;
    }
    ok = ok && hipblasLtMatrixLayoutCreate(&P.la, HIP_R_16F, L.in, L.out, L.in) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&P.lb, HIP_R_16F, L.in, rows, L.in) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&P.ld, HIP_R_32F, L.out, rows, L.out) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulHeuristicResult_t res{};
    int n = 0;
    if (ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
        const uint64_t wmax = tpfm_ctx::LT_WS;
        ok = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wmax,
                                                   sizeof wmax) == HIPBLAS_STATUS_SUCCESS &&
             hipblasLtMatmulAlgoGetHeuristic(c->lt, P.md, P.la, P.lb, P.ld, P.ld, pref, 1, &res, &n) ==
                 HIPBLAS_STATUS_SUCCESS &&
             n >= 1 && res.workspaceSize <= tpfm_ctx::LT_WS;
        (void) hipblasLtMatmulPreferenceDestroy(pref);
    } else {
        ok = false;
    }
    if (ok) {
        P.algo = res.algo;
        P.ws = res.workspaceSize;
    }
    c->lt_plans[key] = P;  // destroyed with the others; an unusable plan is erased below
    if (!ok) {
        tpfm_ctx::LtPlan &Q = c->lt_plans[key];
        if (Q.md) (void) hipblasLtMatmulDescDestroy(Q.md);
        if (Q.la) (void) hipblasLtMatrixLayoutDestroy(Q.la);
        if (Q.lb) (void) hipblasLtMatrixLayoutDestroy(Q.lb);
        if (Q.ld) (void) hipblasLtMatrixLayoutDestroy(Q.ld);
        c->lt_plans.erase(key);
    }
    return ok;
}

// y[rows][L.out] (+ gate, residual, activation, operand copy) = X[rows][L.in] L.W^T + L.b
bool linear(tpfm_ctx *c, const tpfm_ctx::Lin &L, const void *X, int rows, float *Y, void *Ya, bool ya16, int act,
            const float *gate = nullptr, int64_t gstride = 0, const float *res = nullptr) {
    EncConvParams p{};
    p.A = L.W;
    p.X = X;
    p.Y = Y;
    p.Ya = Ya;
    p.ya_f16 = ya16 ? 1 : 0;
    p.bias = L.b;
    p.res = res;
    p.leaky = act;
    p.gate = gate;
    p.gstride = gstride;
    p.H = 1;
    p.W = rows;
    p.IC = L.in;
    p.OC = L.out;
    p.KH = p.KW = 1;
    p.stride = 1;
    p.pad = 0;
    p.OH = 1;
    p.OW = rows;
    p.ws = c->ws;
    if (L.f16) {
        // bias only, f32 output: the library's epilogue writes Y
        const bool direct = Y && !Ya && act == 0 && !gate && !res;
        auto it = c->lt_plans.find(std::make_tuple(rows, L.out, L.in, direct));
        if (direct && (it == c->lt_plans.end() || it->second.bias != (L.b != nullptr)))
            it = c->lt_plans.find(std::make_tuple(rows, L.out, L.in, false));
        if (it != c->lt_plans.end()) {
            const tpfm_ctx::LtPlan &P = it->second;
            const bool dir = std::get<3>(it->first);
            if (dir && P.bias) {
                // the plan's shape is shared by layers with their own biases
                const void *bp = L.b;
                if (hipblasLtMatmulDescSetAttribute(P.md, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof bp) !=
                    HIPBLAS_STATUS_SUCCESS) {
                    c->err = "linear: setting the hipBLASLt bias pointer failed";
                    return false;
                }
            }
            float *D = dir ? Y : c->ws;
            const float alpha = 1.0f, beta = 0.0f;
            const hipblasStatus_t e = hipblasLtMatmul(c->lt, P.md, &alpha, L.W, P.la, X, P.lb, &beta, D, P.ld, D,
                                                      P.ld, &P.algo, c->lt_ws, P.ws, c->stream);
            if (e != HIPBLAS_STATUS_SUCCESS) {
                c->err = ffmt("linear: hipblasLtMatmul failed (status %d)", (int) e);
                return false;
            }
            return dir || c->hip_ok(launch_enc_epilogue(p, c->stream), "linear epilogue");
        }
    }
    p.ksplit = lin_splits(rows, L.out, L.in);
    return c->hip_ok(launch_enc_conv(p, L.f16, c->stream), "linear");
}

// the f32 product X W^T of an f16 linear into ws on its hipBLASLt plan (no
// bias, no epilogue): 1 done, 0 the layer has no plan, -1 error
int lt_product(tpfm_ctx *c, const tpfm_ctx::Lin &L, const void *X, int rows) {
    if (!L.f16) return 0;
    const auto it = c->lt_plans.find(std::make_tuple(rows, L.out, L.in, false));
    if (it == c->lt_plans.end()) return 0;
    const tpfm_ctx::LtPlan &P = it->second;
    const float alpha = 1.0f, beta = 0.0f;
    const hipblasStatus_t e = hipblasLtMatmul(c->lt, P.md, &alpha, L.W, P.la, X, P.lb, &beta, c->ws, P.ld, c->ws,
                                              P.ld, &P.algo, c->lt_ws, P.ws, c->stream);
    if (e != HIPBLAS_STATUS_SUCCESS) {
        c->err = ffmt("linear: hipblasLtMatmul failed (status %d)", (int) e);
        return -1;
    }
    return 1;
}

// c_embed(cond) into clin, from the condition rows in cond_a: the same for
// every ODE step of a chunk, so it runs once per chunk
bool enqueue_cond_embed(tpfm_ctx *c) {
    return linear(c, c->cemb, c->cond_a, c->B * c->T, c->clin, nullptr, false, 0);
}

// the CFG-batched forward on device buffers: x60 (f32 [T][dim_w]) and clin
// (c_embed(cond), f32 [B*T][H]) are in place; v (f32 [B*T][dim_w]) is the result
bool enqueue_forward(tpfm_ctx *c, float t) {
    const tpfm_config &g = c->cfg;
    const int H = g.dim_h, T = c->T, R = c->B * T;
    hipStream_t st = c->stream;
    // t embedding: GLIDE features cos / sin(t f_k) (src/fmt.cpp:168-174, the
    // f_k table made on the host as there), two GEMVs
    if (!c->hip_ok(launch_fmt_tfreq(c->tfk, t, g.t_freq_dim / 2, c->tf, st), "t_freq") ||
        !c->hip_ok(launch_enc_linear(c->t0w, c->t0b, c->tf, H, g.t_freq_dim, c->t0_16, c->te0, st), "t_embed") ||
        !c->hip_ok(launch_fmt_silu(c->te0, H, st), "silu") ||
        !c->hip_ok(launch_enc_linear(c->t2w, c->t2b, c->te0, H, H, c->t2_16, c->te, st), "t_embed"))
        return false;
    // c = c_embed(cond) + t_emb; the adaLN layers read silu(c)
    const bool sc16 = c->mods.f16;
    if (!c->hip_ok(launch_fmt_cond(c->clin, c->te, R, H, c->sc_a, sc16, st), "cond")) return false;
    // x = x_embed(x60) + pos, shared by the branches
    if (!c->hip_ok(launch_fmt_convert(c->x60, T, g.dim_w, g.dim_w, c->x60_a, c->xemb.f16, st), "x60") ||
        !linear(c, c->xemb, c->x60_a, T, c->x1, nullptr, false, 0) ||
        !c->hip_ok(launch_fmt_xpos(c->x1, c->pos, T, H, c->B, c->x, st), "pos"))
        return false;
    // all adaLN modulations at once: block i's shift/scale/gate at columns 6H i .. of mod
    const int64_t ms = c->mods.out;
    if (!linear(c, c->mods, c->sc_a, R, c->mod, nullptr, false, 0)) return false;
    const float *fmd = c->mod + c->blocks.size() * 6 * (size_t) H;  // the final layer's shift / scale
    // x += gate * (X L.W^T + L.b), then h_a = modulate(norm(x)) with the
    // shift / scale at columns sh, sc of nmd: one launch after the library
    // product, or the linear's own epilogue and the norm
    auto residual_norm = [&](const tpfm_ctx::Lin &L, const void *X, const float *gate, const float *nmd, int sh,
                             int sc, bool out16) -> bool {
        const int r = lt_product(c, L, X, R);
        if (r < 0) return false;
        if (r == 1)
            return c->hip_ok(launch_fmt_res_ln_mod(c->ws, L.b, gate, ms, c->x, nmd, ms, sh, sc, R, H, g.ln_eps,
                                                   c->h_a, out16, st),
                             "residual + norm");
        return linear(c, L, X, R, c->x, nullptr, false, 0, gate, ms, c->x) &&
               c->hip_ok(launch_fmt_ln_mod(c->x, nmd, ms, sh, sc, R, H, g.ln_eps, c->h_a, out16, st), "norm");
    };
    // the first block's attention norm (the later norms follow the residual
    // updates that precede them)
    if (!c->blocks.empty() &&
        !c->hip_ok(launch_fmt_ln_mod(c->x, c->mod, ms, 0, H, R, H, g.ln_eps, c->h_a, c->blocks[0].qkv.f16, st),
                   "norm"))
        return false;
    for (size_t i = 0; i < c->blocks.size(); i++) {
        const auto &Bk = c->blocks[i];
        const float *md = c->mod + i * 6 * (size_t) H;
        const bool last = i + 1 == c->blocks.size();
        // attention branch, then the MLP branch's norm
        if (!linear(c, Bk.qkv, c->h_a, R, c->qkv, nullptr, false, 0) ||
            !c->hip_ok(launch_fmt_attn(c->qkv, c->B, T, H, g.n_heads, g.attn_window, c->o_a, Bk.proj.f16, st),
                       "attention") ||
            !residual_norm(Bk.proj, c->o_a, md + 2 * H, md, 3 * H, 4 * H, Bk.fc1.f16))
            return false;
        // MLP branch, then the next block's attention norm (the final layer's norm after the last)
        const float *nmd = last ? fmd : md + 6 * (size_t) H;
        const bool n16 = last ? c->fin_lin.f16 : c->blocks[i + 1].qkv.f16;
        if (!linear(c, Bk.fc1, c->h_a, R, nullptr, c->m1_a, Bk.fc2.f16, 2) ||
            !residual_norm(Bk.fc2, c->m1_a, md + 5 * H, nmd, 0, H, n16))
            return false;
    }
    // final head (its norm came with the last block's residual update)
    if (c->blocks.empty() &&
        !c->hip_ok(launch_fmt_ln_mod(c->x, fmd, ms, 0, H, R, H, g.ln_eps, c->h_a, c->fin_lin.f16, st), "norm"))
        return false;
    if (!linear(c, c->fin_lin, c->h_a, R, c->v, nullptr, false, 0)) return false;
    return true;
}

}  // namespace

extern "C" {

void tpfm_default_config(tpfm_config *g) {
    if (!g) return;
    g->dim_h = 1024;
    g->depth = 8;
    g->n_heads = 8;
    g->dim_w = 512;
    g->dim_a = 512;
    g->dim_e = 7;
    g->chunk_frames = 50;
    g->prev_frames = 10;
    g->attn_window = 2;
    g->t_freq_dim = 256;
    g->nfe = 10;
    g->mlp_ratio = 4.0f;
    g->ln_eps = 1e-6f;
    g->a_cfg = 2.0f;
    g->e_cfg = 1.0f;
    g->r_cfg = 1.0f;
}

static tpfm_ctx *tpfm_create_body(int device, const char *ftype, const tpfm_config *cfg) {
    if (!ftype || (strcmp(ftype, "f32") != 0 && strcmp(ftype, "f16") != 0) || !cfg) {
        fprintf(stderr, "tpfm_create: ftype must be f32 or f16, and a config is needed\n");
        return nullptr;
    }
    const tpfm_config &g = *cfg;
    const int mlp = (int) ((float) g.dim_h * g.mlp_ratio);
    if (g.dim_h <= 0 || g.n_heads <= 0 || g.dim_h % g.n_heads != 0 || g.dim_h / g.n_heads > 256 ||
        g.dim_h % 32 != 0 || g.dim_w % 32 != 0 || g.t_freq_dim % 32 != 0 || mlp % 32 != 0 || g.attn_window < 0 ||
        g.attn_window > 7 || g.depth < 0 || g.dim_a <= 0 || g.dim_e < 0 || g.chunk_frames <= 0 ||
        g.prev_frames < 0 || g.nfe < 2 || g.dim_h > 4096) {
        fprintf(stderr, "tpfm_create: unsupported FMT configuration\n");
        return nullptr;
    }
    tpfm_ctx *c = new tpfm_ctx();
    c->device = device;
    c->f16 = strcmp(ftype, "f16") == 0;
    c->cfg = g;
    c->T = g.chunk_frames + g.prev_frames;
    c->CD = g.dim_w + g.dim_a + g.dim_e;
    c->CDp = round32(c->CD);
    c->MLP = mlp;
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "tpfm_create: no HIP device %d\n", device);
        c->device = -1;
        delete c;
        return nullptr;
    }
    const int half = g.t_freq_dim / 2;
    c->t_freqs.resize((size_t) half);
    for (int k = 0; k < half; k++)
        c->t_freqs[(size_t) k] = (float) exp(-log(10000.0) * (double) k / (double) half);
    make_tensor_list(c);
    return c;
}

void tpfm_destroy(tpfm_ctx *c) { delete c; }

const char *tpfm_last_error(const tpfm_ctx *c) { return c ? c->err.c_str() : "no context"; }

const char *tpfm_weight_name(const tpfm_ctx *c, int i, int64_t *n, int *is_matrix) {
    if (!c || i < 0 || i >= (int) c->tensors.size()) return nullptr;
    const auto &t = c->tensors[(size_t) i];
    int64_t e = 1;
    for (auto d : t.second) e *= d;
    if (n) *n = e;
    if (is_matrix) *is_matrix = t.second.size() >= 2 ? 1 : 0;
    return t.first.c_str();
}

static int tpfm_set_weight_body(tpfm_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    if (!check(c)) return -1;
    if (!name || !data || n <= 0) {
        c->err = "tpfm_set_weight: null name/data or empty tensor";
        return -1;
    }
    const std::vector<int64_t> *shape = nullptr;
    for (const auto &t : c->tensors)
        if (t.first == name) shape = &t.second;
    if (!shape) {
        c->err = ffmt("tpfm_set_weight: unknown FMT tensor %s", name);
        return -1;
    }
    int64_t want = 1;
    for (auto d : *shape) want *= d;
    if (want != n) {
        c->err = ffmt("tpfm_set_weight: %s has %lld elements, expected %lld", name, (long long) n, (long long) want);
        return -1;
    }
    FTensor t;
    t.data.assign(data, data + n);
    t.flags = flags;
    c->host[name] = std::move(t);
    c->prepared = false;
    return 0;
}

static int tpfm_prepare_body(tpfm_ctx *c) {
    if (!check(c)) return -1;
    c->free_all();
    c->prepared = false;
    const tpfm_config &g = c->cfg;
    const int H = g.dim_h, T = c->T, R = c->B * T;
    c->blocks.assign((size_t) g.depth, tpfm_ctx::Block{});
    {
        const FTensor *w0 = c->need("t_embedder.mlp.0.weight"), *b0 = c->need("t_embedder.mlp.0.bias"),
                      *w2 = c->need("t_embedder.mlp.2.weight"), *b2 = c->need("t_embedder.mlp.2.bias"),
                      *pe = c->need("pos_embed");
        if (!w0 || !b0 || !w2 || !b2 || !pe) return -1;
        c->t0_16 = c->kept16(*w0);
        c->t2_16 = c->kept16(*w2);
        c->t0w = c->upload(c->dev_value(*w0));
        c->t0b = c->upload(b0->data);
        c->t2w = c->upload(c->dev_value(*w2));
        c->t2b = c->upload(b2->data);
        c->pos = c->upload(c->dev_value(*pe));
        if (!c->t0w || !c->t0b || !c->t2w || !c->t2b || !c->pos) return -1;
    }
    if (!make_lin(c, c->cemb, "c_embedder", H, c->CD, c->CDp) ||
        !make_lin(c, c->xemb, "x_embedder.proj", H, g.dim_w, g.dim_w))
        return -1;
    for (int i = 0; i < g.depth; i++) {
        auto &B = c->blocks[(size_t) i];
        const std::string b = ffmt("blocks.%d", i);
        if (!make_lin(c, B.qkv, b + ".attn.qkv", 3 * H, H, H) || !make_lin(c, B.proj, b + ".attn.proj", H, H, H) ||
            !make_lin(c, B.fc1, b + ".mlp.fc1", c->MLP, H, H) || !make_lin(c, B.fc2, b + ".mlp.fc2", H, c->MLP, c->MLP))
            return -1;
    }
    {
        std::vector<std::pair<std::string, int>> mb;
        for (int i = 0; i < g.depth; i++) mb.push_back({ffmt("blocks.%d.adaLN_modulation.1", i), 6 * H});
        mb.push_back({"decoder.adaLN_modulation.1", 2 * H});
        // (silu(c) is one operand buffer for every adaLN layer: they share a type)
        if (!make_lin_stack(c, c->mods, mb, H, H) || !make_lin(c, c->fin_lin, "decoder.linear", g.dim_w, H, H))
            return -1;
    }
    auto F = [&](size_t n) { return (float *) c->dalloc(n * 4); };
    auto A = [&](size_t n) { return c->dalloc(n * 4); };  // operand buffers sized for f32
    c->tf = F((size_t) g.t_freq_dim);
    c->tfk = c->upload(c->t_freqs);
    c->te0 = F((size_t) H);
    c->te = F((size_t) H);
    c->cond_f = F((size_t) R * c->CD);
    c->cond_a = A((size_t) R * c->CDp);
    c->clin = F((size_t) R * H);
    c->sc_a = A((size_t) R * H);
    c->x60 = F((size_t) T * g.dim_w);
    c->x60_a = A((size_t) T * g.dim_w);
    c->x1 = F((size_t) T * H);
    c->x = F((size_t) R * H);
    c->mod = F((size_t) R * c->mods.out);
    c->h_a = A((size_t) R * std::max(H, g.dim_w));
    c->qkv = F((size_t) R * 3 * H);
    c->o_a = A((size_t) R * H);
    c->m1_a = A((size_t) R * c->MLP);
    c->v = F((size_t) R * g.dim_w);
    {
        size_t wsn = 1;
        // f16 linears may run their product on hipBLASLt into ws
        const char *ev = getenv("TPFM_BLASLT");
        const bool use_lt = c->f16 && !(ev && ev[0] == '0');
        auto need_ws = [&](const tpfm_ctx::Lin &L, int rows) {
            const int k = lin_splits(rows, L.out, L.in);
            if (k > 1) wsn = std::max(wsn, (size_t) k * rows * L.out);
            if (use_lt && L.f16) wsn = std::max(wsn, (size_t) rows * L.out);
        };
        need_ws(c->cemb, R);
        need_ws(c->xemb, T);
        need_ws(c->mods, R);
        need_ws(c->fin_lin, R);
        for (const auto &B : c->blocks) {
            need_ws(B.qkv, R);
            need_ws(B.proj, R);
            need_ws(B.fc1, R);
            need_ws(B.fc2, R);
        }
        c->ws = F(wsn);
        if (use_lt) {
            if (!c->lt && hipblasLtCreate(&c->lt) != HIPBLAS_STATUS_SUCCESS) {
                c->lt = nullptr;
                c->err = "hipblasLtCreate failed";
                return -1;
            }
            c->lt_ws = c->dalloc(tpfm_ctx::LT_WS);
            if (!c->lt_ws) return -1;
            auto plan = [&](const tpfm_ctx::Lin &L, int rows, bool direct) {
                if (L.f16) (void) lt_plan(c, L, rows, direct);
            };
            plan(c->cemb, R, true);
            plan(c->xemb, T, true);
            plan(c->mods, R, true);
            plan(c->fin_lin, R, true);
            for (const auto &B : c->blocks) {
                plan(B.qkv, R, true);
                plan(B.proj, R, false);
                plan(B.fc1, R, false);
                plan(B.fc2, R, false);
            }
        }
    }
    c->h_cond.assign((size_t) 3 * T * c->CD, 0.0f);
    c->h_x60.assign((size_t) T * g.dim_w, 0.0f);
    if (!c->tf || !c->tfk || !c->te0 || !c->te || !c->cond_f || !c->cond_a || !c->clin || !c->sc_a || !c->x60 || !c->x60_a ||
        !c->x1 || !c->x || !c->mod || !c->h_a || !c->qkv || !c->o_a || !c->m1_a || !c->v || !c->ws)
        return -1;
    c->prepared = true;
    return 0;
}

static int tpfm_forward_body(tpfm_ctx *c, const float *x60, const float *cond, float t, float *v_out) {
    if (!check(c)) return -1;
    if (!c->prepared) {
        c->err = "FMT not prepared";
        return -1;
    }
    if (!x60 || !cond || !v_out) {
        c->err = "tpfm_forward: null buffer";
        return -1;
    }
    const int T = c->T, R = c->B * T, D = c->cfg.dim_w;
    hipStream_t st = c->stream;
    if (!c->hip_ok(hipMemcpyAsync(c->x60, x60, (size_t) T * D * 4, hipMemcpyHostToDevice, st), "x60") ||
        !c->hip_ok(hipMemcpyAsync(c->cond_f, cond, (size_t) R * c->CD * 4, hipMemcpyHostToDevice, st), "cond") ||
        !c->hip_ok(launch_fmt_convert(c->cond_f, R, c->CD, c->CDp, c->cond_a, c->cemb.f16, st), "cond"))
        return -1;
    if (!enqueue_cond_embed(c) || !enqueue_forward(c, t)) return -1;
    if (!c->hip_ok(hipMemcpyAsync(v_out, c->v, (size_t) R * D * 4, hipMemcpyDeviceToHost, st), "v") ||
        !c->hip_ok(hipStreamSynchronize(st), "forward sync"))
        return -1;
    return 0;
}

static int tpfm_sample_chunk_body(tpfm_ctx *c, const float *wr, const float *prev_x, const float *prev_wa,
                      const float *cond_audio, int emotion, const float *x0, float *motion_out) {
    if (!check(c)) return -1;
    if (!c->prepared) {
        c->err = "FMT not prepared";
        return -1;
    }
    const tpfm_config &g = c->cfg;
    const int T = c->T, P = g.prev_frames, CF = g.chunk_frames, D = g.dim_w, DA = g.dim_a, CD = c->CD;
    if (!wr || (P > 0 && (!prev_x || !prev_wa)) || !cond_audio || !x0 || !motion_out) {
        c->err = "tpfm_sample_chunk: null buffer";
        return -1;
    }
    // condition rows [wr | wa | we] per branch and frame (src/pipeline.cpp:22-36)
    // (host staging kept by the context: a chunk allocates nothing)
    std::vector<float> &cond = c->h_cond, &x60 = c->h_x60;
    cond.assign((size_t) 3 * T * CD, 0.0f);
    x60.resize((size_t) T * D);
    for (int b = 0; b < 3; b++)
        for (int f = 0; f < T; f++) {
            float *row = cond.data() + ((size_t) b * T + f) * CD;
            memcpy(row, wr, (size_t) D * 4);
            const float *wa = f < P ? prev_wa + (size_t) f * DA : cond_audio + (size_t) (f - P) * DA;
            if (!(b == 0 && f >= P)) memcpy(row + D, wa, (size_t) DA * 4);
            if (b == 1 && emotion >= 0 && emotion < g.dim_e) row[D + DA + emotion] = 1.0f;
        }
    if (P > 0) memcpy(x60.data(), prev_x, (size_t) P * D * 4);
    memcpy(x60.data() + (size_t) P * D, x0, (size_t) CF * D * 4);
    hipStream_t st = c->stream;
    const int R = 3 * T;
    if (!c->hip_ok(hipMemcpyAsync(c->x60, x60.data(), x60.size() * 4, hipMemcpyHostToDevice, st), "x60") ||
        !c->hip_ok(hipMemcpyAsync(c->cond_f, cond.data(), cond.size() * 4, hipMemcpyHostToDevice, st), "cond") ||
        !c->hip_ok(launch_fmt_convert(c->cond_f, R, CD, c->CDp, c->cond_a, c->cemb.f16, st), "cond"))
        return -1;
    // torch linspace(0, 1, nfe) in f32 (src/pipeline.cpp:12-13)
    auto ode_t = [&](int i) { return (float) ((double) i / (double) (g.nfe - 1)); };
    if (!enqueue_cond_embed(c)) return -1;
    for (int s = 0; s < g.nfe - 1; s++) {
        if (!enqueue_forward(c, ode_t(s))) return -1;
        const float dt = ode_t(s + 1) - ode_t(s);
        if (!c->hip_ok(launch_fmt_euler(c->v, c->x60, T, P, D, g.a_cfg, g.e_cfg, dt, st), "euler")) return -1;
    }
    if (!c->hip_ok(hipMemcpyAsync(motion_out, c->x60 + (size_t) P * D, (size_t) CF * D * 4, hipMemcpyDeviceToHost,
                                  st),
                   "motion") ||
        !c->hip_ok(hipStreamSynchronize(st), "sample sync"))
        return -1;
    return 0;
}


// ---- entry points that allocate host memory, exception-safe

tpfm_ctx *tpfm_create(int device, const char *ftype, const tpfm_config *cfg) {
    return guarded((void *) nullptr, [&] { return tpfm_create_body(device, ftype, cfg); });
}

int tpfm_set_weight(tpfm_ctx *c, const char *name, const float *data, int64_t n, int flags) {
    return guarded(c, [&] { return tpfm_set_weight_body(c, name, data, n, flags); });
}

int tpfm_prepare(tpfm_ctx *c) {
    return guarded(c, [&] { return tpfm_prepare_body(c); });
}

int tpfm_forward(tpfm_ctx *c, const float *x60, const float *cond, float t, float *v_out) {
    return guarded(c, [&] { return tpfm_forward_body(c, x60, cond, t, v_out); });
}

int tpfm_sample_chunk(tpfm_ctx *c, const float *wr, const float *prev_x, const float *prev_wa,
                      const float *cond_audio, int emotion, const float *x0, float *motion_out) {
    return guarded(c, [&] { return tpfm_sample_chunk_body(c, wr, prev_x, prev_wa, cond_audio, emotion, x0, motion_out); });
}

}  // extern "C"
