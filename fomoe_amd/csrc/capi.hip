// capi.hip — host side of the C-ABI declared in include/gpu.h.
//
// One context = one device, one stream, lazily grown scratch. Every launch is
// argument-checked on the host against the shapes the kernels cover before
// anything reaches the device.
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "common.h"
#include "gpu.h"
#include "kernels.h"
#include "moe.h"
#include "prefill.h"
#include "context.h"

using namespace fo;

// ------------------------------------------------------------------ no-allocation scratch
// The device scratch of gpu_moe_layer_noalloc: one static array, held until
// the process ends. Contexts always run on device 0 (gpu_init selects it, as
// the reference's does), so one copy of the array is in use. Host code never
// passes `fo_noalloc_scratch` itself to a kernel (in host code the name is a
// host-side stand-in): its device address is looked up with
// hipGetSymbolAddress in gpu_init, with device 0 current, and kept in
// g_noalloc_ptr.
static constexpr size_t kNoAllocBytes = 1u << 20;   // GPU_MOE_NOALLOC_SCRATCH_BYTES
static_assert(kNoAllocBytes == GPU_MOE_NOALLOC_SCRATCH_BYTES, "header and library agree");
static __device__ __align__(256) uint8_t fo_noalloc_scratch[kNoAllocBytes];
static void *g_noalloc_ptr;

static hipError_t noalloc_setup() {
    if (g_noalloc_ptr) return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(fo_noalloc_scratch));
    if (e != hipSuccess || !p) return e != hipSuccess ? e : hipErrorInvalidSymbol;
    g_noalloc_ptr = p;
    return hipSuccess;
}

extern "C" {

gpu_ctx_t *gpu_init(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return nullptr;
    gpu_ctx *c = new gpu_ctx();
    c->device = 0;
    hipDeviceProp_t prop;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        delete c;
        return nullptr;
    }
    c->n_cu = prop.multiProcessorCount;
    c->hbm = prop.totalGlobalMem;
    snprintf(c->arch, sizeof c->arch, "%s", prop.gcnArchName);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {   // code objects are gfx950-only
        delete c;
        return nullptr;
    }
    bool ok = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreate(&c->ev0) == hipSuccess && hipEventCreate(&c->ev1) == hipSuccess &&
              hipMalloc((void **)&c->logits, 1024 * sizeof(float)) == hipSuccess &&
              hipMalloc((void **)&c->counter, 256) == hipSuccess &&
              hipMalloc((void **)&c->ids, 64 * sizeof(int32_t)) == hipSuccess &&
              hipMalloc((void **)&c->weights, 64 * sizeof(float)) == hipSuccess &&
              hipMemset(c->counter, 0, 256) == hipSuccess &&
              hipMemset(c->ids, 0, 64 * sizeof(int32_t)) == hipSuccess &&
              noalloc_setup() == hipSuccess &&
              hipDeviceSynchronize() == hipSuccess;
    if (!ok) {
        gpu_free(c);
        return nullptr;
    }
    return c;
}

void gpu_free(gpu_ctx_t *c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    void *bufs[] = {c->logits, c->counter, c->ids, c->weights, c->xq_h, c->xq_act, c->act,
                    c->act2, c->vec_in, c->vec_out, c->staging, c->pf_logits, c->pf_ids,
                    c->pf_w, c->pf_pairpos, c->pf_pairtok, c->pf_tiles, c->pf_ntiles,
                    c->pf_act, c->pf_outp, c->pf_xsum, c->pf_rsplit, c->sh_act, c->sh_ys,
                    c->pf_ys};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    for (int b = 0; b < 2; b++) {
        if (c->pin[b]) (void)hipHostFree(c->pin[b]);
        if (c->pin_ev[b]) (void)hipEventDestroy(c->pin_ev[b]);
    }
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char *gpu_last_error(gpu_ctx_t *c) { return c ? c->err.c_str() : "null context"; }

int gpu_device_info(gpu_ctx_t *ctx, int *n_cu, uint64_t *hbm, char *arch, int arch_len) {
    if (!ctx) return -1;
    if (n_cu) *n_cu = ctx->n_cu;
    if (hbm) *hbm = ctx->hbm;
    if (arch && arch_len > 0) snprintf(arch, (size_t)arch_len, "%s", ctx->arch);
    return 0;
}

void *gpu_alloc(gpu_ctx_t *ctx, uint64_t bytes) {
    if (!ctx || bytes == 0) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        fail(ctx, -2, "hipMalloc(%llu) failed", (unsigned long long)bytes);
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

void gpu_dealloc(gpu_ctx_t *ctx, void *p) {
    if (ctx && p) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(p);
    }
}

int gpu_upload(gpu_ctx_t *ctx, void *d, const void *h, uint64_t bytes) {
    if (!ctx || (!d && bytes) || (!h && bytes)) return fail(ctx, -1, "gpu_upload: null pointer");
    if (!bytes) return 0;
    HIPC(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIPC(hipStreamSynchronize(ctx->stream));
    return 0;
}

int gpu_download(gpu_ctx_t *ctx, void *h, const void *d, uint64_t bytes) {
    if (!ctx || (!d && bytes) || (!h && bytes)) return fail(ctx, -1, "gpu_download: null pointer");
    if (!bytes) return 0;
    HIPC(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIPC(hipStreamSynchronize(ctx->stream));
    return 0;
}

int gpu_sync(gpu_ctx_t *ctx) {
    if (!ctx) return -1;
    HIPC(hipStreamSynchronize(ctx->stream));
    return 0;
}

int gpu_timer_start(gpu_ctx_t *ctx) {
    if (!ctx) return -1;
    HIPC(hipEventRecord(ctx->ev0, ctx->stream));
    return 0;
}

float gpu_timer_stop(gpu_ctx_t *ctx) {
    if (!ctx) return -1.f;
    float ms = -1.f;
    if (hipEventRecord(ctx->ev1, ctx->stream) != hipSuccess ||
        hipEventSynchronize(ctx->ev1) != hipSuccess ||
        hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) != hipSuccess)
        return -1.f;
    return ms;
}

// ------------------------------------------------------------------ kernels
int gpu_dequantize(gpu_ctx_t *ctx, int type, const void *src, float *dst, int64_t n) {
    if (!ctx || !src || !dst || n <= 0) return fail(ctx, -1, "gpu_dequantize: bad argument");
    const int bv = fomoe_block_values(type);
    if (bv == 0 || n % bv) return fail(ctx, -1, "gpu_dequantize: type %d / n %lld", type, (long long)n);
    HIPC(launch_dequant(type, (const uint8_t *)src, dst, n, ctx->stream));
    return 0;
}

// Prepare the activation(s) of a matvec into ctx->xq_act.
static int prep_x(gpu_ctx_t *ctx, int type, const float *x, uint64_t x_stride, int K, int n_vec,
                  uint64_t &stride_out) {
    const int gsz = gsz_of(type);
    stride_out = xq_stride(K, gsz);
    HIPC(ensure(ctx->xq_act, ctx->xq_act_cap, stride_out * (size_t)n_vec));
    HIPC(launch_xprep(gsz, x, x_stride, K, n_vec, ctx->xq_act, stride_out, ctx->stream));
    return 0;
}

int gpu_matvec_q_batched(gpu_ctx_t *ctx, int type, const void *W, uint64_t mat_stride, int n_mats,
                         const float *x, uint64_t x_stride, float *y, uint64_t y_stride, int M, int K) {
    if (!ctx || !W || !x || !y || M <= 0 || K <= 0 || n_mats <= 0)
        return fail(ctx, -1, "gpu_matvec_q: bad argument");
    if (!matvec_type(type)) return fail(ctx, -1, "gpu_matvec_q: unsupported type %d", type);
    if (K % fomoe_block_values(type) || (kquant(type) && K % 256) || K > 16384)
        return fail(ctx, -1, "gpu_matvec_q: K=%d not supported for type %d", K, type);
    const uint64_t rb = fomoe_row_bytes(type, K);
    if (matvec_self_prep(type, rb, K, x_stride)) {   // the kernel prepares x itself: one launch
        MatvecArgs a{(const uint8_t *)W, mat_stride, rb, nullptr, 0, y, y_stride, n_mats, M, K, x, x_stride};
        HIPC(launch_matvec(type, a, ctx->stream, ctx->n_cu));
        return 0;
    }
    uint64_t xs = 0;
    int rc = prep_x(ctx, type, x, x_stride, K, x_stride ? n_mats : 1, xs);
    if (rc) return rc;
    MatvecArgs a{(const uint8_t *)W, mat_stride, rb, ctx->xq_act, x_stride ? xs : 0, y, y_stride, n_mats, M, K,
                 nullptr, 0};
    HIPC(launch_matvec(type, a, ctx->stream, ctx->n_cu));
    return 0;
}

int gpu_matvec_q(gpu_ctx_t *ctx, int type, const void *W, const float *x, float *y, int M, int K) {
    return gpu_matvec_q_batched(ctx, type, W, 0, 1, x, 0, y, 0, M, K);
}

// ------------------------------------------------------------------ MoE
static int check_layer(gpu_ctx_t *ctx, const gpu_moe_layer_t *L) {
    if (!L || !L->router || !L->experts) return fail(ctx, -1, "moe layer: null pointer");
    if (L->n_embd <= 0 || L->n_embd % 256 || L->n_embd > 8192)
        return fail(ctx, -1, "moe layer: n_embd %d (multiple of 256, <= 8192)", L->n_embd);
    if (L->inter <= 0 || L->inter % 256 || L->inter > 8192)
        return fail(ctx, -1, "moe layer: inter %d (multiple of 256, <= 8192)", L->inter);
    if (L->n_experts <= 0 || L->n_experts > 1024 || L->k <= 0 || L->k > 16 || L->k > L->n_experts)
        return fail(ctx, -1, "moe layer: n_experts %d / k %d", L->n_experts, L->k);
    if (!layer_type(L->gate_type) || L->up_type != L->gate_type || !layer_type(L->down_type))
        return fail(ctx, -1, "moe layer: types gate %d up %d down %d", L->gate_type, L->up_type,
                    L->down_type);
    const uint64_t gs = fomoe_row_bytes(L->gate_type, L->n_embd) * (uint64_t)L->inter;
    const uint64_t ds = fomoe_row_bytes(L->down_type, L->inter) * (uint64_t)L->n_embd;
    if (L->gate_size < gs || L->up_size < gs || L->expert_stride < L->gate_size + L->up_size + ds)
        return fail(ctx, -1, "moe layer: blob sizes too small for the shapes");
    if (L->shared) {   // its own types and intermediate size (reference include/model.h:104-108)
        const int Fs = L->shared_inter;
        if (Fs <= 0 || Fs % 256 || Fs > 8192)
            return fail(ctx, -1, "moe layer: shared_inter %d (multiple of 256, <= 8192)", Fs);
        if (!layer_type(L->shared_gate_type) || !layer_type(L->shared_up_type) || !layer_type(L->shared_down_type))
            return fail(ctx, -1, "moe layer: shared types gate %d up %d down %d", L->shared_gate_type,
                        L->shared_up_type, L->shared_down_type);
        if (L->shared_gate_size < fomoe_row_bytes(L->shared_gate_type, L->n_embd) * (uint64_t)Fs ||
            L->shared_up_size < fomoe_row_bytes(L->shared_up_type, L->n_embd) * (uint64_t)Fs)
            return fail(ctx, -1, "moe layer: shared gate/up sizes too small for the shapes");
    }
    return 0;
}

// Size every scratch buffer a layer needs (outside any graph capture).
static int size_layer(gpu_ctx_t *ctx, const gpu_moe_layer_t *L) {
    const int n_tot = L->k + (L->shared ? 1 : 0);   // slot k: a fused shared expert
    HIPC(ensure(ctx->xq_h, ctx->xq_h_cap, xq_stride(L->n_embd, gsz_of(L->gate_type))));
    HIPC(ensure(ctx->act, ctx->act_cap, sizeof(float) * (size_t)n_tot * L->inter));
    HIPC(ensure(ctx->xq_act, ctx->xq_act_cap, xq_stride(L->inter, gsz_of(L->down_type)) * (size_t)n_tot));
    if (L->shared) {
        HIPC(ensure(ctx->sh_act, ctx->sh_act_cap, sizeof(float) * (size_t)L->shared_inter));
        HIPC(ensure(ctx->sh_ys, ctx->sh_ys_cap, sizeof(float) * (size_t)L->n_embd));
    }
    return 0;
}

// Shapes the three-kernel path (moe.hip) covers; others take the general path.
static bool fast_layer(const gpu_moe_layer_t *L) {
    const int dslot = L->down_type == GGML_TYPE_Q8_0 ? 32 : 64;
    const int n_tot = L->k + (L->shared ? 1 : 0);
    return L->n_embd % 512 == 0 && L->n_embd <= 8192 && L->inter / dslot <= 64 && n_tot <= 16;
}

static constexpr int kSharedW = 32;   // weights[32] holds the shared-expert weight

// Device scratch of one layer call: the context's grown buffers, or the
// carve-up of the static no-allocation area.
struct LayerScratch {
    float *logits;       // [1024]
    unsigned *counter;   // general router's completion counter (zero between calls)
    int32_t *ids;        // [64]
    float *weights;      // [64]
    uint8_t *xq_h;       // prepared h
    uint8_t *xq_act;     // n_tot prepared activations
    float *act;          // [n_tot x F] fp32 activations (general path)
    float *sh_act;       // [F_s] shared-expert activation
    float *sh_ys;        // [H] weighted shared-expert output
};

static LayerScratch ctx_scratch(gpu_ctx_t *ctx) {
    return LayerScratch{ctx->logits, ctx->counter, ctx->ids, ctx->weights, ctx->xq_h, ctx->xq_act, ctx->act,
                        ctx->sh_act, ctx->sh_ys};
}

// The shared expert's description for its roles (shared.h); w: where the
// layer's kernels leave the shared-expert weight.
static SharedArgs shared_args(const LayerScratch &sc, const gpu_moe_layer_t *L, const float *w) {
    SharedArgs s{};
    if (!L->shared) return s;
    const int H = L->n_embd, Fs = L->shared_inter;
    s.blob = (const uint8_t *)L->shared;
    s.gate_type = L->shared_gate_type;
    s.up_type = L->shared_up_type;
    s.down_type = L->shared_down_type;
    s.up_off = L->shared_gate_size;
    s.down_off = L->shared_gate_size + L->shared_up_size;
    s.gate_rb = fomoe_row_bytes(s.gate_type, H);
    s.up_rb = fomoe_row_bytes(s.up_type, H);
    s.down_rb = fomoe_row_bytes(s.down_type, Fs);
    s.F = Fs;
    s.H = H;
    s.act = sc.sh_act;
    s.w = w;
    s.ys = sc.sh_ys;
    s.down_rpw = shared_down_rpw(Fs);
    s.down_waves = 4;
    return s;
}

// How the fast path runs the shared expert: fused = with the routed experts'
// types and intermediate size it is expert slot k of the layer kernels;
// down-only = only its down projection differs in type (the usual GGUF mix):
// its gate/up ride in k_expand as slot k (fp32 activation kept) and its down
// projection runs on the matvec kernel; otherwise the shared-expert kernels
// of shared.h.
enum SharedMode { kSharedNone, kSharedFused, kSharedDownOnly, kSharedOwn };

static SharedMode shared_mode(const gpu_moe_layer_t *L) {
    if (!L->shared) return kSharedNone;
    const bool gu = L->shared_inter == L->inter && L->shared_gate_type == L->gate_type &&
                    L->shared_up_type == L->up_type && L->shared_gate_size == L->gate_size &&
                    L->shared_up_size == L->up_size;
    if (gu && L->shared_down_type == L->down_type) return kSharedFused;
    if (gu && matvec_self_prep(L->shared_down_type, fomoe_row_bytes(L->shared_down_type, L->inter), L->inter, 0))
        return kSharedDownOnly;
    return kSharedOwn;
}

static int enqueue_layer_fast(gpu_ctx_t *ctx, const LayerScratch &sc, const gpu_moe_layer_t *L,
                              const float *in, float *out, int flags, const float *norm_w) {
    const int H = L->n_embd, F = L->inter;
    const int dg = gsz_of(L->down_type);
    const uint64_t xs = xq_stride(F, dg);
    const SharedMode mode = shared_mode(L);
    const uint8_t *base = (const uint8_t *)L->experts, *sh = (const uint8_t *)L->shared;
    const uint8_t *sh2 = (mode == kSharedFused || mode == kSharedDownOnly) ? sh : nullptr;   // slot k of k_expand
    float *shared_w = sc.weights + kSharedW;
    RouteArgs ra{L->router, L->router_bias, in, norm_w, L->eps, L->n_experts, H, sc.logits,
                 sc.xq_h, gsz_of(L->gate_type), L->shared_gate_vec, L->shared ? shared_w : nullptr};
    HIPC(launch_route(ra, ctx->stream));
    if (mode == kSharedOwn) HIPC(launch_shared(shared_args(sc, L, nullptr), in, norm_w, L->eps, ctx->stream));
    const bool fused = mode == kSharedFused;
    ReduceArgs da{sc.ids, sc.weights, L->shared ? shared_w : nullptr, L->k, base, L->expert_stride,
                  L->gate_size + L->up_size, fused ? sh : nullptr, L->shared_gate_size + L->shared_up_size, F, H,
                  fomoe_row_bytes(L->down_type, F), sc.xq_act, xs,
                  (flags & GPU_MOE_RESIDUAL) ? in : nullptr, out, mode == kSharedOwn ? sc.sh_ys : nullptr,
                  -1, nullptr, nullptr};
    // a down projection with activation groups of 32 (Q4_K, Q5_K) beside Q4_K
    // gate/up at H = 4096: the 16-row gate/up kernel leaves fp32 activations
    // and the down kernel prepares its groups from them
    const bool f32act = dg == 32 && L->gate_type == GGML_TYPE_Q4_K && H == 4096 &&
                        reduce_takes_tile(L->down_type, da);
    ExpandArgs ea{sc.logits, L->n_experts, L->k, sc.ids, sc.weights, base, L->expert_stride,
                  L->gate_size, sh2, L->shared_gate_size, F, H, fomoe_row_bytes(L->gate_type, H),
                  sc.xq_h, sc.xq_act, xs, dg, (mode == kSharedDownOnly || f32act) ? sc.act : nullptr,
                  f32act ? 1 : 0};
    HIPC(launch_expand(L->gate_type, ea, ctx->stream, ctx->n_cu));
    if (f32act) da.act_f32 = sc.act;
    if (mode == kSharedDownOnly) {
        const int sdt = L->shared_down_type;
        if (reduce_takes_shared_type(L->down_type, da, sdt)) {   // one more block in k_reduce_tile
            da.shared = sh;
            da.sh_type = sdt;
            da.sh_act = sc.act + (size_t)L->k * F;
        } else {   // ys = down_s . act_s on the matvec kernel, unweighted
            MatvecArgs ma{sh + L->shared_gate_size + L->shared_up_size, 0, fomoe_row_bytes(sdt, F), nullptr, 0,
                          sc.sh_ys, 0, 1, H, F, sc.act + (size_t)L->k * F, 0};
            HIPC(launch_matvec(sdt, ma, ctx->stream, ctx->n_cu));
            da.ys = sc.sh_ys;
        }
    }
    HIPC(launch_reduce(L->down_type, da, ctx->stream, ctx->n_cu));
    return 0;
}

static int enqueue_layer(gpu_ctx_t *ctx, const LayerScratch &sc, const gpu_moe_layer_t *L,
                         const float *in, float *out, int flags) {
    const int H = L->n_embd, F = L->inter, k = L->k;
    const float *norm_w = (flags & GPU_MOE_NORM) ? L->norm_w : nullptr;
    if ((flags & GPU_MOE_NORM) && !norm_w) return fail(ctx, -1, "moe layer: GPU_MOE_NORM without norm_w");
    const bool fast = fast_layer(L);
    if (fast) {
        const int rc = enqueue_layer_fast(ctx, sc, L, in, out, flags, norm_w);
        if (!rc) ctx->last_fast = true;
        return rc;
    }
    ctx->last_fast = false;
    RouterArgs ra{L->router, L->router_bias, in, norm_w, L->eps, L->n_experts, H, L->k,
                  sc.logits, sc.counter, sc.ids, sc.weights, L->shared_gate_vec};
    HIPC(launch_router(ra, sc.xq_h, gsz_of(L->gate_type), ctx->stream));
    const uint8_t *base = (const uint8_t *)L->experts;
    if (L->shared) {   // the shared expert first: the router leaves its weight at weights[k]
        const SharedArgs sa = shared_args(sc, L, sc.weights + k);
        HIPC(launch_shared(sa, in, norm_w, L->eps, ctx->stream));
    }
    GateUpArgs ga{sc.ids, k, base, L->expert_stride, 0, L->gate_size, F, H,
                  fomoe_row_bytes(L->gate_type, H), in, norm_w, L->eps, sc.act};
    HIPC(launch_gateup(L->gate_type, ga, sc.xq_h, ctx->stream, ctx->n_cu));
    const int gsz = gsz_of(L->down_type);
    const uint64_t xs = xq_stride(F, gsz);
    HIPC(launch_xprep(gsz, sc.act, (uint64_t)F, F, k, sc.xq_act, xs, ctx->stream));
    DownArgs da{sc.ids, sc.weights, k, base, L->expert_stride, L->gate_size + L->up_size,
                L->shared ? sc.sh_ys : nullptr, sc.act, H, F,
                fomoe_row_bytes(L->down_type, F), (flags & GPU_MOE_RESIDUAL) ? in : nullptr, out};
    HIPC(launch_down(L->down_type, da, sc.xq_act, xs, ctx->stream, ctx->n_cu));
    return 0;
}

int gpu_moe_layer(gpu_ctx_t *ctx, const gpu_moe_layer_t *L, const float *in, float *out, int flags) {
    if (!ctx || !in || !out) return fail(ctx, -1, "gpu_moe_layer: null pointer");
    int rc = check_layer(ctx, L);
    if (!rc) rc = size_layer(ctx, L);
    if (!rc) rc = enqueue_layer(ctx, ctx_scratch(ctx), L, in, out, flags);
    if (!rc) {
        ctx->last_k = L->k;
        ctx->last_ids = ctx->ids;
        ctx->last_weights = ctx->weights;
    }
    return rc;
}

// Byte layout of the no-allocation scratch for one layer (256-byte aligned
// pieces); returns the bytes needed.
static size_t noalloc_layout(const gpu_moe_layer_t *L, uint8_t *base, LayerScratch *sc) {
    const int n_tot = L->k + (L->shared ? 1 : 0);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t *p = base + off;
        off += (bytes + 255) & ~(size_t)255;
        return p;
    };
    uint8_t *logits = take(1024 * sizeof(float)), *counter = take(256), *ids = take(64 * sizeof(int32_t)),
            *weights = take(64 * sizeof(float)), *xq_h = take(xq_stride(L->n_embd, gsz_of(L->gate_type))),
            *xq_act = take(xq_stride(L->inter, gsz_of(L->down_type)) * (size_t)n_tot),
            *act = take(sizeof(float) * (size_t)n_tot * L->inter),
            *sh_act = take(L->shared ? sizeof(float) * (size_t)L->shared_inter : 0),
            *sh_ys = take(L->shared ? sizeof(float) * (size_t)L->n_embd : 0);
    if (sc)
        *sc = LayerScratch{(float *)logits, (unsigned *)counter, (int32_t *)ids, (float *)weights, xq_h, xq_act,
                           (float *)act, (float *)sh_act, (float *)sh_ys};
    return off;
}

int gpu_moe_layer_noalloc(gpu_ctx_t *ctx, const gpu_moe_layer_t *L, const float *in, float *out, int flags) {
    if (!ctx || !in || !out) return fail(ctx, -1, "gpu_moe_layer_noalloc: null pointer");
    if (int rc = check_layer(ctx, L)) return rc;
    const size_t need = noalloc_layout(L, nullptr, nullptr);
    if (need > kNoAllocBytes)
        return fail(ctx, -1, "gpu_moe_layer_noalloc: layer needs %zu bytes of scratch, the static area holds %zu",
                    need, kNoAllocBytes);
    uint8_t *base = (uint8_t *)g_noalloc_ptr;
    if (!base) return fail(ctx, -2, "gpu_moe_layer_noalloc: scratch address unknown");
    LayerScratch sc;
    noalloc_layout(L, base, &sc);
    // the area keeps the previous call's contents: the general router's
    // completion counter must start at zero (a kernel fill, not a memset node)
    if (!fast_layer(L)) HIPC(launch_zero_u32(sc.counter, 64, ctx->stream));
    const int rc = enqueue_layer(ctx, sc, L, in, out, flags);
    if (!rc) {
        ctx->last_k = L->k;
        ctx->last_ids = sc.ids;
        ctx->last_weights = sc.weights;
    }
    return rc;
}

int gpu_moe_last_routing(gpu_ctx_t *ctx, int32_t *ids, float *w, float *shared_w) {
    if (!ctx || ctx->last_k <= 0) return fail(ctx, -1, "no routing recorded");
    float tmp[64];
    HIPC(hipStreamSynchronize(ctx->stream));
    if (ids) HIPC(hipMemcpy(ids, ctx->last_ids, sizeof(int32_t) * ctx->last_k, hipMemcpyDeviceToHost));
    HIPC(hipMemcpy(tmp, ctx->last_weights, sizeof(float) * (kSharedW + 1), hipMemcpyDeviceToHost));
    if (w) memcpy(w, tmp, sizeof(float) * ctx->last_k);
    if (shared_w) *shared_w = ctx->last_fast ? tmp[kSharedW] : tmp[ctx->last_k];
    return 0;
}

int gpu_router_topk(gpu_ctx_t *ctx, const float *router, const float *bias, const float *x,
                    const float *norm_w, float eps, int E, int H, int k, int32_t *ids, float *w) {
    if (!ctx || !router || !x || !ids || !w) return fail(ctx, -1, "gpu_router_topk: null pointer");
    if (E <= 0 || E > 1024 || k <= 0 || k > 16 || k > E || H <= 0 || H % 256 || H > 8192)
        return fail(ctx, -1, "gpu_router_topk: E %d k %d H %d", E, k, H);
    RouterArgs ra{router, bias, x, norm_w, eps, E, H, k, ctx->logits, ctx->counter, ids, w, nullptr};
    HIPC(launch_router(ra, nullptr, 32, ctx->stream));
    return 0;
}

int gpu_moe_stack_decode(gpu_ctx_t *ctx, const gpu_moe_layer_t *layers, int n_layers, float *x,
                         int n_steps) {
    if (!ctx || !layers || !x || n_layers <= 0 || n_steps < 0)
        return fail(ctx, -1, "gpu_moe_stack_decode: bad argument");
    for (int l = 0; l < n_layers; l++) {
        int rc = check_layer(ctx, &layers[l]);
        if (!rc) rc = size_layer(ctx, &layers[l]);
        if (rc) return rc;
        if (!layers[l].norm_w) return fail(ctx, -1, "gpu_moe_stack_decode: layer %d has no norm_w", l);
    }
    if (n_steps == 0) return 0;
    // The captured graph bakes in every pointer it was built from: the layer
    // descriptors, x and the context's scratch. A call with the same ones
    // replays it; anything else captures anew.
    const LayerScratch sc = ctx_scratch(ctx);
    std::vector<uint8_t> key(sizeof(gpu_moe_layer_t) * (size_t)n_layers + sizeof x + sizeof sc);
    memcpy(key.data(), layers, sizeof(gpu_moe_layer_t) * (size_t)n_layers);
    memcpy(key.data() + sizeof(gpu_moe_layer_t) * (size_t)n_layers, &x, sizeof x);
    memcpy(key.data() + sizeof(gpu_moe_layer_t) * (size_t)n_layers + sizeof x, &sc, sizeof sc);
    if (!ctx->graph_exec || key != ctx->graph_key) {
        if (ctx->graph_exec) {
            (void)hipGraphExecDestroy(ctx->graph_exec);
            ctx->graph_exec = nullptr;
        }
        ctx->graph_key.clear();
        HIPC(hipStreamSynchronize(ctx->stream));
        HIPC(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        int rc = 0;
        for (int l = 0; l < n_layers && !rc; l++)
            rc = enqueue_layer(ctx, sc, &layers[l], x, x, GPU_MOE_NORM | GPU_MOE_RESIDUAL);
        hipGraph_t g = nullptr;
        hipError_t ce = hipStreamEndCapture(ctx->stream, &g);
        if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
        if (ce != hipSuccess) return fail(ctx, -2, "graph capture failed: %s", hipGetErrorString(ce));
        hipError_t ie = hipGraphInstantiate(&ctx->graph_exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ie != hipSuccess) return fail(ctx, -2, "graph instantiate failed: %s", hipGetErrorString(ie));
        ctx->graph_key = std::move(key);
    }
    for (int s = 0; s < n_steps; s++) HIPC(hipGraphLaunch(ctx->graph_exec, ctx->stream));
    ctx->last_k = layers[n_layers - 1].k;
    ctx->last_ids = ctx->ids;
    ctx->last_weights = ctx->weights;
    return 0;
}

// ------------------------------------------------------------------ reference lifecycle
// The reference's whole-model entry points (include/gpu.h:19-66). This library
// has no whole-model forward, so each returns the reference's "not available"
// result and the reference's caller falls back to its CPU path
// (model.c:411-431, inference.c:425-431, main.c:569-580, 951-956).
void gpu_register_buffers(gpu_ctx_t *, void **, int, uint64_t) {}
void gpu_unregister_buffers(gpu_ctx_t *, void **, int) {}
int gpu_upload_model(gpu_ctx_t *ctx, const void *) {
    return fail(ctx, -1, "gpu_upload_model: no whole-model forward in this library");
}
void gpu_set_ram_cache_mb(gpu_ctx_t *ctx, int mb) { if (ctx) ctx->ram_cache_mb = mb; }
void gpu_set_vram_cache_mb(gpu_ctx_t *ctx, int mb) { if (ctx) ctx->vram_cache_mb = mb; }
float *gpu_forward(gpu_ctx_t *ctx, void *, int, int) {
    fail(ctx, -1, "gpu_forward: no whole-model forward in this library");
    return nullptr;
}
void gpu_reset_state(gpu_ctx_t *) {}
int gpu_seed_vram_cache(gpu_ctx_t *ctx, void *, const char *) {
    return fail(ctx, -1, "gpu_seed_vram_cache: no expert cache tiers in this library");
}
void gpu_enable_expert_freq(gpu_ctx_t *) {}
const uint32_t *gpu_get_expert_freq(gpu_ctx_t *) { return nullptr; }
void gpu_get_expert_dims(gpu_ctx_t *, int *n_layers, int *n_experts) {
    if (n_layers) *n_layers = 0;
    if (n_experts) *n_experts = 0;
}
void gpu_get_pingpong_relay_stats(gpu_ctx_t *, uint64_t *handoffs, uint64_t *payload, uint64_t *d2h,
                                  uint64_t *h2d, uint64_t *dma) {
    uint64_t *outs[] = {handoffs, payload, d2h, h2d, dma};
    for (uint64_t *p : outs)
        if (p) *p = 0;
}

// ------------------------------------------------------------------ legacy FFN
// Reference gpu_kernels.hip:8385-8488: same argument checks and -1 fallbacks
// (limits MAX_EXPERTS 10, MAX_N_EMBD 4096, MAX_INTERMEDIATE 2048,
// MAX_EXPERT_STRIDE 12 MiB at gpu_kernels.hip:438-441).
int gpu_expert_ffn(gpu_ctx_t *ctx, const float *h, void **expert_buffers, const float *scores,
                   int n_experts, int n_embd, int inter, uint64_t gate_size, uint64_t up_size,
                   uint64_t stride, int gate_type, int up_type, int down_type, float *ffn_out) {
    if (!ctx) return -1;
    if (n_experts > 10 || n_embd > 4096 || inter > 2048 || stride > 12ull * 1024 * 1024) return -1;
    if (!kquant(gate_type) || !kquant(up_type) || !kquant(down_type)) return -1;
    if (!h || !ffn_out || n_embd <= 0 || inter <= 0 || n_embd % 256 || inter % 256) return -1;
    if (n_experts <= 0) {
        memset(ffn_out, 0, sizeof(float) * (size_t)n_embd);
        return 0;
    }
    if (!expert_buffers || !scores) return -1;
    hipStream_t s = ctx->stream;
    const int H = n_embd, F = inter, n = n_experts;
    if (ensure(ctx->staging, ctx->staging_cap, (size_t)n * stride) != hipSuccess ||
        ensure(ctx->vec_in, ctx->vec_in_cap, sizeof(float) * (size_t)H) != hipSuccess ||
        ensure(ctx->vec_out, ctx->vec_out_cap, sizeof(float) * (size_t)H) != hipSuccess ||
        ensure(ctx->act, ctx->act_cap, sizeof(float) * (size_t)n * F) != hipSuccess ||
        ensure(ctx->act2, ctx->act2_cap, sizeof(float) * (size_t)n * F) != hipSuccess ||
        // room for two prepared copies of h at the widest layout (gsz 16):
        // gate and up may be prepared in different group sizes below
        ensure(ctx->xq_h, ctx->xq_h_cap, 2 * xq_stride(H, 16)) != hipSuccess ||
        ensure(ctx->xq_act, ctx->xq_act_cap, xq_stride(F, 16) * (size_t)n) != hipSuccess)
        return fail(ctx, -1, "gpu_expert_ffn: scratch allocation failed");
    if (hipMemcpyAsync(ctx->vec_in, h, sizeof(float) * H, hipMemcpyHostToDevice, s) != hipSuccess)
        return -1;
    for (int e = 0; e < n; e++)
        if (!expert_buffers[e] ||
            hipMemcpyAsync(ctx->staging + (size_t)e * stride, expert_buffers[e], stride,
                           hipMemcpyHostToDevice, s) != hipSuccess)
            return -1;
    if (hipMemcpyAsync(ctx->weights, scores, sizeof(float) * n, hipMemcpyHostToDevice, s) != hipSuccess)
        return -1;
    const uint64_t rb_g = fomoe_row_bytes(gate_type, H), rb_u = fomoe_row_bytes(up_type, H);
    if (gate_type == up_type) {
        const int gsz = gsz_of(gate_type);
        if (launch_xprep(gsz, ctx->vec_in, 0, H, 1, ctx->xq_h, xq_stride(H, gsz), s) != hipSuccess) return -1;
        GateUpArgs ga{nullptr, n, ctx->staging, stride, 0, gate_size, F, H, rb_g, ctx->vec_in, nullptr, 0.f,
                      ctx->act};
        if (launch_gateup(gate_type, ga, ctx->xq_h, s, ctx->n_cu) != hipSuccess) return -1;
    } else {
        // gate and up in different formats: two batched matvecs + SiLU*up
        uint8_t *xg = ctx->xq_h, *xu = ctx->xq_h + xq_stride(H, 16);
        if (launch_xprep(gsz_of(gate_type), ctx->vec_in, 0, H, 1, xg, 0, s) != hipSuccess ||
            launch_xprep(gsz_of(up_type), ctx->vec_in, 0, H, 1, xu, 0, s) != hipSuccess)
            return -1;
        MatvecArgs mg{ctx->staging, stride, rb_g, xg, 0, ctx->act, (uint64_t)F, n, F, H};
        MatvecArgs mu{ctx->staging + gate_size, stride, rb_u, xu, 0, ctx->act2, (uint64_t)F, n, F, H};
        if (launch_matvec(gate_type, mg, s, ctx->n_cu) != hipSuccess ||
            launch_matvec(up_type, mu, s, ctx->n_cu) != hipSuccess ||
            launch_silu_mul(ctx->act, ctx->act2, (int64_t)n * F, s) != hipSuccess)
            return -1;
    }
    const int gsz = gsz_of(down_type);
    const uint64_t xs = xq_stride(F, gsz);
    if (launch_xprep(gsz, ctx->act, (uint64_t)F, F, n, ctx->xq_act, xs, s) != hipSuccess) return -1;
    DownArgs da{nullptr, ctx->weights, n, ctx->staging, stride, gate_size + up_size, nullptr,
                ctx->act, H, F, fomoe_row_bytes(down_type, F), nullptr, ctx->vec_out};
    if (launch_down(down_type, da, ctx->xq_act, xs, s, ctx->n_cu) != hipSuccess) return -1;
    if (hipMemcpyAsync(ffn_out, ctx->vec_out, sizeof(float) * H, hipMemcpyDeviceToHost, s) != hipSuccess)
        return -1;
    if (hipStreamSynchronize(s) != hipSuccess) return -1;
    return 0;
}

// ------------------------------------------------------------------ synthetic
int gpu_synth_f32(gpu_ctx_t *ctx, uint64_t seed, uint64_t stream, float std, float *out, int64_t n) {
    if (!ctx || !out || n <= 0) return fail(ctx, -1, "gpu_synth_f32: bad argument");
    HIPC(launch_synth_f32(seed, stream, std, out, n, ctx->stream));
    return 0;
}

int gpu_synth_quant(gpu_ctx_t *ctx, int type, uint64_t seed, uint64_t stream0, uint64_t step, float std,
                    int64_t M, int64_t K, int n_mats, void *dst, uint64_t dst_stride) {
    if (!ctx || !dst || M <= 0 || K <= 0 || K % 256 || n_mats <= 0)
        return fail(ctx, -1, "gpu_synth_quant: bad argument");
    if (!layer_type(type)) return fail(ctx, -1, "gpu_synth_quant: type %d", type);
    HIPC(launch_synth_quant(type, seed, stream0, step, std, M, K, n_mats, (uint8_t *)dst, dst_stride,
                            ctx->stream));
    return 0;
}

void gpu_synth_zipf_bias(uint64_t seed, uint64_t stream, int n, double s, float *bias) {
    if (n <= 0 || !bias) return;
    auto mix = [](uint64_t z) {
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    const uint64_t G = 0x9E3779B97F4A7C15ull;
    const uint64_t key = mix(seed * G + mix(stream + 0x632BE59BD9B4E019ull));
    std::vector<int> perm((size_t)n);
    for (int i = 0; i < n; i++) perm[(size_t)i] = i;
    for (int i = n - 1; i > 0; i--) {
        const int j = (int)(mix(key + ((uint64_t)i + 1) * G) % (uint64_t)(i + 1));
        std::swap(perm[(size_t)i], perm[(size_t)j]);
    }
    for (int r = 0; r < n; r++) bias[perm[(size_t)r]] = (float)(-s * log((double)(r + 1)));
}


// ------------------------------------------------------------------ prefill
int gpu_moe_prefill(gpu_ctx_t *ctx, const gpu_moe_layer_t *L, const uint16_t *d_x, int n_tokens,
                    float *d_out, int flags) {
    if (!ctx) return -1;
    if (int rc = check_layer(ctx, L)) return rc;
    if (!d_x || !d_out || n_tokens <= 0) return fail(ctx, -1, "moe prefill: null buffer or n_tokens %d", n_tokens);
    if (flags & ~GPU_MOE_RESIDUAL) return fail(ctx, -1, "moe prefill: flags %d (only GPU_MOE_RESIDUAL)", flags);
    if (!fo::prefill_types_ok(L->gate_type, L->up_type, L->down_type))
        return fail(ctx, -1, "moe prefill: types gate %d up %d down %d (gate/up Q4_K/Q6_K, or both Q5_K or "
                             "both Q8_0; down Q4_K, Q5_K, Q6_K or Q8_0)", L->gate_type, L->up_type, L->down_type);
    // a shared expert whose gate/up types or F_s differ runs as a one-expert
    // pass of its own (every token routed to it), whose output the routed
    // pass combines; one that differs in its down type only (the usual GGUF
    // mix) shares the routed gate/up GEMM and gets a down launch of its own
    const bool own = L->shared && (L->shared_inter != L->inter || L->shared_gate_type != L->gate_type ||
                                   L->shared_up_type != L->up_type);
    const bool down_own = L->shared && !own && L->shared_down_type != L->down_type;
    if ((own || down_own) && !fo::prefill_types_ok(L->shared_gate_type, L->shared_up_type, L->shared_down_type))
        return fail(ctx, -1, "moe prefill: shared-expert types gate %d up %d down %d", L->shared_gate_type,
                    L->shared_up_type, L->shared_down_type);
    const int T = n_tokens, E = L->n_experts, k = L->k, H = L->n_embd, F = L->inter;
    if (E > 1023) return fail(ctx, -1, "moe prefill: n_experts %d > 1023", E);
    if (L->gate_type == GGML_TYPE_Q4_K) {   // its gate/up rows move by direct 16-byte global->LDS loads
        auto a16 = [](uint64_t v) { return v % 16 == 0; };
        if (!a16((uintptr_t)L->experts) || !a16(L->expert_stride) || !a16(L->gate_size) ||
            (L->shared && !own && (!a16((uintptr_t)L->shared) || !a16(L->shared_gate_size))))
            return fail(ctx, -1, "moe prefill: Q4_K gate/up blobs must be 16-byte aligned "
                                 "(experts, shared, expert_stride, gate sizes)");
    }
    // the grouping table holds n_experts x ceil(tokens/32) words: larger
    // batches run as consecutive chunks (the results per token are the same)
    const int Tc = std::min(T, (16384 / E) * 32);
    if (own && L->shared_gate_type == GGML_TYPE_Q4_K &&
        ((uintptr_t)L->shared % 16 || L->shared_gate_size % 16))
        return fail(ctx, -1, "moe prefill: a Q4_K shared blob and its gate size must be 16-byte aligned");
    const bool sh = L->shared != nullptr && !own;
    const int Fs = own ? L->shared_inter : F;
    const size_t P = (size_t)fo::prefill_pairs(Tc, k, sh);
    const int max_tiles = fo::prefill_max_tiles(Tc, k, E, sh);
    HIPC(ensure(ctx->pf_logits, ctx->pf_logits_cap, sizeof(float) * (size_t)Tc * E));
    HIPC(ensure(ctx->pf_ids, ctx->pf_ids_cap, sizeof(int32_t) * (size_t)T * k));
    HIPC(ensure(ctx->pf_w, ctx->pf_w_cap, sizeof(float) * (size_t)T * (k + 1)));
    HIPC(ensure(ctx->pf_pairpos, ctx->pf_pairpos_cap, sizeof(int32_t) * (size_t)Tc * (k + 1)));
    HIPC(ensure(ctx->pf_pairtok, ctx->pf_pairtok_cap, sizeof(int32_t) * P));
    const size_t tcap = (size_t)std::max(max_tiles, fo::prefill_max_tiles(Tc, 1, 1, false));
    HIPC(ensure(ctx->pf_tiles, ctx->pf_tiles_cap, sizeof(int32_t) * 8 * tcap));   // tiles, then double tiles
    HIPC(ensure(ctx->pf_ntiles, ctx->pf_ntiles_cap, 256));
    const size_t Pact = std::max(P * F, (size_t)Tc * Fs);   // activation elements of either pass
    HIPC(ensure(ctx->pf_act, ctx->pf_act_cap, 2 * sizeof(uint16_t) * Pact));
    if (own)   // the shared pass's output [Tc x H] (its down rows, pairs in token order)
        HIPC(ensure(ctx->pf_ys, ctx->pf_ys_cap, sizeof(float) * (size_t)Tc * H));
    HIPC(ensure(ctx->pf_outp, ctx->pf_outp_cap, sizeof(float) * P * H));
    HIPC(ensure(ctx->pf_rsplit, ctx->pf_rsplit_cap, sizeof(uint16_t) * fo::prefill_router_ws_elems(E, Tc, H)));
    // xsum [Tc x H/32] fp32, then x16 [Tc x H] fp16, then xexp [Tc] int32, then pexp [P] int32
    const size_t xs_bytes = sizeof(float) * (size_t)Tc * (H / 32), x16_bytes = 2 * (size_t)Tc * H;
    HIPC(ensure(ctx->pf_xsum, ctx->pf_xsum_cap, xs_bytes + x16_bytes + sizeof(int32_t) * ((size_t)Tc + P)));
    fo::PrefillArgs a{};
    a.E = E; a.k = k; a.H = H; a.F = F;
    a.gate_type = L->gate_type; a.up_type = L->up_type; a.down_type = L->down_type;
    a.router = L->router; a.router_bias = L->router_bias;
    a.experts = (const uint8_t *)L->experts; a.stride = L->expert_stride;
    a.gate_size = L->gate_size; a.up_size = L->up_size;
    a.shared = sh ? (const uint8_t *)L->shared : nullptr;
    a.sh_gate_size = L->shared_gate_size; a.sh_up_size = L->shared_up_size;
    a.ys = own ? ctx->pf_ys : nullptr;
    a.sh_down_type = down_own ? L->shared_down_type : -1;
    a.shared_gate_vec = L->shared_gate_vec;
    a.residual = (flags & GPU_MOE_RESIDUAL) ? 1 : 0;
    a.logits = ctx->pf_logits; a.pairpos = ctx->pf_pairpos;
    a.pair_tok = ctx->pf_pairtok; a.tiles = ctx->pf_tiles; a.n_tiles = ctx->pf_ntiles;
    a.dtiles = ctx->pf_tiles + 4 * tcap;
    a.act_hi = ctx->pf_act; a.act_lo = ctx->pf_act + Pact; a.outp = ctx->pf_outp;
    a.xsum = ctx->pf_xsum;
    a.x16 = (uint16_t *)((uint8_t *)ctx->pf_xsum + xs_bytes);
    a.xexp = (int32_t *)((uint8_t *)ctx->pf_xsum + xs_bytes + x16_bytes);
    a.pexp = a.xexp + Tc;
    a.rsplit = ctx->pf_rsplit;
    for (int t0 = 0; t0 < T; t0 += Tc) {
        const int n = std::min(Tc, T - t0);
        a.T = n;
        a.max_tiles = fo::prefill_max_tiles(n, k, E, sh);
        a.x = d_x + (size_t)t0 * H;
        a.out = d_out + (size_t)t0 * H;
        a.ids = ctx->pf_ids + (size_t)t0 * k;
        a.w = ctx->pf_w + (size_t)t0 * (k + 1);
        if (own) {   // shared pass first: ys = shared_ffn(x) for the chunk's tokens
            fo::PrefillArgs b = a;
            b.E = 1; b.k = 1; b.F = Fs;
            b.gate_type = L->shared_gate_type; b.up_type = L->shared_up_type; b.down_type = L->shared_down_type;
            b.one_expert = 1;             // no router or combine: the down rows are ys in token order
            b.xprep_ready = 0;            // this chunk's tokens are prepared here
            b.router = nullptr; b.router_bias = nullptr;
            b.experts = (const uint8_t *)L->shared;
            const uint64_t sds = fomoe_row_bytes(L->shared_down_type, Fs) * (uint64_t)H;
            b.stride = (L->shared_gate_size + L->shared_up_size + sds + 15) & ~(uint64_t)15;
            b.gate_size = L->shared_gate_size; b.up_size = L->shared_up_size;
            b.shared = nullptr; b.shared_gate_vec = nullptr; b.ys = nullptr; b.sh_down_type = -1;
            b.residual = 0; b.out = nullptr; b.outp = ctx->pf_ys;
            b.max_tiles = fo::prefill_max_tiles(n, 1, 1, false);
            HIPC(fo::launch_prefill(b, ctx->stream));
        }
        // the shared pass prepared these tokens' fp16 rows for Q4_K gate/up
        a.xprep_ready = own && L->shared_gate_type == GGML_TYPE_Q4_K && L->shared_up_type == GGML_TYPE_Q4_K;
        HIPC(fo::launch_prefill(a, ctx->stream));
    }
    ctx->pf_T = T;
    ctx->pf_k = k;
    return 0;
}

int gpu_moe_prefill_routing(gpu_ctx_t *ctx, int32_t *ids, float *weights) {
    if (!ctx) return -1;
    if (ctx->pf_T <= 0) return fail(ctx, -1, "moe prefill routing: no prefill has run");
    HIPC(hipStreamSynchronize(ctx->stream));
    if (ids) HIPC(hipMemcpy(ids, ctx->pf_ids, sizeof(int32_t) * (size_t)ctx->pf_T * ctx->pf_k, hipMemcpyDeviceToHost));
    if (weights)
        HIPC(hipMemcpy(weights, ctx->pf_w, sizeof(float) * (size_t)ctx->pf_T * (ctx->pf_k + 1), hipMemcpyDeviceToHost));
    return 0;
}

int gpu_f32_to_bf16(gpu_ctx_t *ctx, const float *d_src, uint16_t *d_dst, int64_t n) {
    if (!ctx || !d_src || !d_dst || n <= 0) return fail(ctx, -1, "f32_to_bf16: bad arguments");
    HIPC(fo::launch_f32_to_bf16(d_src, d_dst, n, ctx->stream));
    return 0;
}

}  // extern "C"

// ------------------------------------------------------------------ file staging
constexpr size_t kPinChunk = 32u << 20;

int file_to_device(gpu_ctx *ctx, int fd, uint64_t file_off, uint64_t bytes, uint8_t *dst, uint64_t seg,
                   uint64_t dst_pitch, const char *what) {
    if (seg == 0) return fail(ctx, -1, "%s: empty segment", what);
    for (int b = 0; b < 2; b++) {
        if (!ctx->pin[b]) HIPC(hipHostMalloc((void **)&ctx->pin[b], kPinChunk, hipHostMallocDefault));
        if (!ctx->pin_ev[b]) HIPC(hipEventCreateWithFlags(&ctx->pin_ev[b], hipEventDisableTiming));
    }
    int rc = 0;
    bool used[2] = {false, false};
    uint64_t off = 0;
    for (int b = 0; off < bytes && rc == 0; b ^= 1) {
        const size_t n = (size_t)std::min<uint64_t>(kPinChunk, bytes - off);
        if (used[b] && hipEventSynchronize(ctx->pin_ev[b]) != hipSuccess) { rc = -2; break; }
        size_t got = 0;
        while (got < n) {
            const ssize_t r = pread(fd, ctx->pin[b] + got, n - got, (off_t)(file_off + off + got));
            if (r <= 0) break;
            got += (size_t)r;
        }
        if (got != n) { rc = fail(ctx, -1, "%s: short read at offset %llu", what, (unsigned long long)(file_off + off)); break; }
        // the chunk's pieces, each inside one segment
        for (uint64_t p = 0; p < n && rc == 0;) {
            const uint64_t lb = off + p, s = lb / seg, w = lb % seg;
            const uint64_t len = std::min<uint64_t>(n - p, seg - w);
            if (hipMemcpyAsync(dst + s * dst_pitch + w, ctx->pin[b] + p, len, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
                rc = -2;
            p += len;
        }
        if (rc == 0 && hipEventRecord(ctx->pin_ev[b], ctx->stream) != hipSuccess) rc = -2;
        used[b] = true;
        off += n;
    }
    // copies still in flight read the pinned chunks: drain them on every path
    const hipError_t se = hipStreamSynchronize(ctx->stream);
    if (rc == -2 || se != hipSuccess) return fail(ctx, -2, "%s: device copy failed", what);
    return rc;
}

// ------------------------------------------------------------------ expert store
static_assert(sizeof(gpu_qmoe_header_t) == 64, "qmoe header is 64 bytes on disk");
static_assert(sizeof(gpu_qmoe_layer_entry_t) == 32, "qmoe layer entry is 32 bytes on disk");

extern "C" {

// Header and index of a .qmoe file (reference src/expert_store.c:11-100),
// validated against the file size so that later reads stay inside it.
static bool qmoe_index(const char *path, gpu_qmoe_header_t &h, std::vector<gpu_qmoe_layer_entry_t> &idx,
                       std::string &err) {
    const int fd = path ? open(path, O_RDONLY) : -1;
    if (fd < 0) { err = std::string("qmoe: cannot open ") + (path ? path : "(null)"); return false; }
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && pread(fd, &h, sizeof h, 0) == (ssize_t)sizeof h;
    if (!ok) err = "qmoe: cannot read the header";
    else if (h.magic != GPU_QMOE_MAGIC) { ok = false; err = "qmoe: bad magic"; }
    else if (h.version < GPU_QMOE_VERSION) { ok = false; err = "qmoe: format version < 2"; }
    else if (h.n_moe_layers == 0 || h.n_moe_layers > 65536 || h.n_experts == 0 || h.n_experts > 65536) {
        ok = false; err = "qmoe: bad layer / expert counts";
    }
    if (ok) {
        idx.resize(h.n_moe_layers);
        const size_t bytes = idx.size() * sizeof(gpu_qmoe_layer_entry_t);
        ok = pread(fd, idx.data(), bytes, 64) == (ssize_t)bytes;
        if (!ok) err = "qmoe: truncated layer index";
    }
    const uint64_t index_end = 64 + (uint64_t)h.n_moe_layers * sizeof(gpu_qmoe_layer_entry_t);
    for (size_t l = 0; ok && l < idx.size(); l++) {
        const uint64_t stride = idx[l].expert_stride ? idx[l].expert_stride : h.expert_stride;
        const uint64_t down = idx[l].down_size ? idx[l].down_size : h.expert_down_size;
        if (stride == 0 || stride < h.expert_gate_size + h.expert_up_size + down ||
            idx[l].data_offset < index_end ||
            idx[l].data_offset + (uint64_t)h.n_experts * stride > (uint64_t)st.st_size) {
            ok = false;
            err = "qmoe: layer " + std::to_string(l) + " does not fit the file";
        }
    }
    close(fd);
    return ok;
}

int gpu_qmoe_read_index(const char *path, gpu_qmoe_header_t *hdr, gpu_qmoe_layer_entry_t *layers,
                        int max_layers, const char **err) {
    static thread_local std::string msg;
    gpu_qmoe_header_t h;
    std::vector<gpu_qmoe_layer_entry_t> idx;
    if (!qmoe_index(path, h, idx, msg)) {
        if (err) *err = msg.c_str();
        return -1;
    }
    msg.clear();
    if (err) *err = msg.c_str();
    if (hdr) *hdr = h;
    if (layers)
        for (int l = 0; l < max_layers && l < (int)idx.size(); l++) layers[l] = idx[l];
    return (int)h.n_moe_layers;
}

int gpu_qmoe_upload_layer(gpu_ctx_t *ctx, const char *path, int layer, void *d_dst, uint64_t dst_bytes) {
    if (!ctx || !d_dst) return fail(ctx, -1, "qmoe upload: null context or destination");
    gpu_qmoe_header_t h;
    std::vector<gpu_qmoe_layer_entry_t> idx;
    std::string msg;
    if (!qmoe_index(path, h, idx, msg)) return fail(ctx, -1, "%s", msg.c_str());
    if (layer < 0 || layer >= (int)idx.size()) return fail(ctx, -1, "qmoe upload: layer %d of %zu", layer, idx.size());
    const uint64_t stride = idx[layer].expert_stride ? idx[layer].expert_stride : h.expert_stride;
    const uint64_t total = (uint64_t)h.n_experts * stride;
    if (dst_bytes < total) return fail(ctx, -1, "qmoe upload: destination %llu < %llu bytes",
                                       (unsigned long long)dst_bytes, (unsigned long long)total);
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(ctx, -1, "qmoe upload: cannot open %s", path);
    const int rc = file_to_device(ctx, fd, idx[layer].data_offset, total, (uint8_t *)d_dst, total, 0, "qmoe upload");
    close(fd);
    return rc;
}

int gpu_qmoe_layer_desc(const gpu_qmoe_header_t *h, const gpu_qmoe_layer_entry_t *e, gpu_moe_layer_t *L) {
    if (!h || !e || !L) return -1;
    L->gate_type = L->up_type = (int)h->quant_type;
    L->down_type = e->down_size ? (int)e->down_type : (int)h->quant_type;
    L->gate_size = h->expert_gate_size;
    L->up_size = h->expert_up_size;
    L->expert_stride = e->expert_stride ? e->expert_stride : h->expert_stride;
    return 0;
}

}  // extern "C"
