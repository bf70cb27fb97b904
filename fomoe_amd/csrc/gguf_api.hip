// gguf_api.hip — the gpu_gguf_* entry points of include/gpu.h: the GGUF
// directory (gguf_file.cpp), host reads, uploads into HBM through the
// context's pinned staging, and assembly of one resident MoE layer from a
// model's tensors in the layout the layer kernels read.
#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "context.h"
#include "gguf_file.h"
#include "kernels.h"

struct gpu_gguf {
    fo::GgufFile f;
};

namespace {

thread_local std::string g_open_err;

const fo::GgufTensor *tensor_at(const gpu_gguf *g, int64_t id) {
    return (g && id >= 0 && id < (int64_t)g->f.tensors.size()) ? &g->f.tensors[id] : nullptr;
}

// File, absolute offset and size of a tensor's data, checked against the file.
bool tensor_span(const gpu_gguf *g, const fo::GgufTensor &t, uint64_t &off, std::string &err) {
    if (t.size == 0) { err = "gguf: tensor " + t.name + " has a type of unknown size"; return false; }
    off = g->f.data_offset[t.split] + t.offset;
    if (off < t.offset || off + t.size < off || off + t.size > g->f.file_size[t.split]) {
        err = "gguf: tensor " + t.name + " lies past the end of " + g->f.paths[t.split];
        return false;
    }
    return true;
}

int64_t elements(const fo::GgufTensor &t) {
    int64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; d++) n *= t.dims[d];
    return n;
}

constexpr uint64_t kStoreAlign = 4096;   // expert stride alignment of the .qmoe layout

}  // namespace

extern "C" {

gpu_gguf_t *gpu_gguf_open(const char *path, const char **err) {
    gpu_gguf *g = new gpu_gguf();
    std::string e;
    if (!g->f.open(path, e)) {
        delete g;
        g_open_err = e;
        if (err) *err = g_open_err.c_str();
        return nullptr;
    }
    if (err) *err = "";
    return g;
}

void gpu_gguf_close(gpu_gguf_t *g) { delete g; }

int64_t gpu_gguf_n_tensors(const gpu_gguf_t *g) { return g ? (int64_t)g->f.tensors.size() : -1; }
int64_t gpu_gguf_n_keys(const gpu_gguf_t *g) { return g ? (int64_t)g->f.keys.size() : -1; }
int64_t gpu_gguf_find_tensor(const gpu_gguf_t *g, const char *name) { return g ? g->f.find_tensor(name) : -1; }
int64_t gpu_gguf_find_key(const gpu_gguf_t *g, const char *key) { return g ? g->f.find_key(key) : -1; }

int gpu_gguf_tensor_info(const gpu_gguf_t *g, int64_t id, gpu_gguf_tensor_t *out) {
    const fo::GgufTensor *t = tensor_at(g, id);
    if (!t || !out) return -1;
    out->name = t->name.c_str();
    out->n_dims = t->n_dims;
    out->type = t->type;
    for (int d = 0; d < 4; d++) out->dims[d] = t->dims[d];
    out->offset = t->offset;
    out->size = t->size;
    out->split = t->split;
    out->pad = 0;
    return 0;
}

const char *gpu_gguf_key(const gpu_gguf_t *g, int64_t i, int *type) {
    if (!g || i < 0 || i >= (int64_t)g->f.keys.size()) return nullptr;
    if (type) *type = g->f.values[i].type;
    return g->f.keys[i].c_str();
}

int gpu_gguf_get_int(const gpu_gguf_t *g, const char *key, int64_t *v) {
    const int64_t i = gpu_gguf_find_key(g, key);
    if (i < 0) return -1;
    const fo::GgufValue &x = g->f.values[i];
    switch (x.type) {
        case 0: case 2: case 4: case 7: case 10: if (v) *v = (int64_t)x.u; return 0;
        case 1: case 3: case 5: case 11: if (v) *v = x.i; return 0;
        default: return -1;
    }
}

int gpu_gguf_get_float(const gpu_gguf_t *g, const char *key, double *v) {
    const int64_t i = gpu_gguf_find_key(g, key);
    if (i < 0) return -1;
    const fo::GgufValue &x = g->f.values[i];
    if (x.type == 6 || x.type == 12) { if (v) *v = x.f; return 0; }
    int64_t iv;
    if (gpu_gguf_get_int(g, key, &iv) == 0) { if (v) *v = (double)iv; return 0; }
    return -1;
}

const char *gpu_gguf_get_str(const gpu_gguf_t *g, const char *key) {
    const int64_t i = gpu_gguf_find_key(g, key);
    return (i >= 0 && g->f.values[i].type == 8) ? g->f.values[i].s.c_str() : nullptr;
}

int gpu_gguf_get_arr(const gpu_gguf_t *g, const char *key, int *elem_type, uint64_t *n, const void **data) {
    const int64_t i = gpu_gguf_find_key(g, key);
    if (i < 0 || g->f.values[i].type != 9) return -1;
    const fo::GgufValue &x = g->f.values[i];
    if (elem_type) *elem_type = x.arr_type;
    if (n) *n = x.arr_n;
    if (data) *data = x.arr_type == 8 ? nullptr : (const void *)x.arr.data();
    return 0;
}

const char *gpu_gguf_get_arr_str(const gpu_gguf_t *g, const char *key, uint64_t j) {
    const int64_t i = gpu_gguf_find_key(g, key);
    if (i < 0 || g->f.values[i].type != 9 || g->f.values[i].arr_type != 8 || j >= g->f.values[i].arr_n)
        return nullptr;
    return g->f.values[i].arr_str[j].c_str();
}

uint64_t gpu_gguf_type_bytes(int type, uint64_t n) { return fo::gguf_type_bytes(type, n); }

int64_t gpu_gguf_read_tensor(const gpu_gguf_t *g, int64_t id, void *h_dst, uint64_t bytes) {
    const fo::GgufTensor *t = tensor_at(g, id);
    uint64_t off;
    std::string err;
    if (!t || !h_dst || bytes < t->size || !tensor_span(g, *t, off, err)) return -1;
    const int fd = open(g->f.paths[t->split].c_str(), O_RDONLY);
    if (fd < 0) return -1;
    uint64_t got = 0;
    while (got < t->size) {
        const ssize_t r = pread(fd, (uint8_t *)h_dst + got, (size_t)std::min<uint64_t>(t->size - got, 1ull << 30),
                                (off_t)(off + got));
        if (r <= 0) break;
        got += (uint64_t)r;
    }
    close(fd);
    return got == t->size ? (int64_t)got : -1;
}

}  // extern "C"

// Scatter a tensor's data into device memory as segments of `seg` bytes at
// dst + i * pitch (plain copy: seg = size, pitch 0).
static int upload_segments(gpu_ctx *ctx, const gpu_gguf *g, const fo::GgufTensor &t, uint8_t *dst, uint64_t seg,
                           uint64_t pitch) {
    uint64_t off;
    std::string err;
    if (!tensor_span(g, t, off, err)) return fail(ctx, -1, "%s", err.c_str());
    const int fd = open(g->f.paths[t.split].c_str(), O_RDONLY);
    if (fd < 0) return fail(ctx, -1, "gguf: cannot open %s", g->f.paths[t.split].c_str());
    const int rc = file_to_device(ctx, fd, off, t.size, dst, seg, pitch, "gguf upload");
    close(fd);
    return rc;
}

extern "C" {

int gpu_gguf_upload_tensor(gpu_ctx_t *ctx, const gpu_gguf_t *g, int64_t id, void *d_dst, uint64_t dst_bytes) {
    if (!ctx) return -1;
    const fo::GgufTensor *t = tensor_at(g, id);
    if (!t || !d_dst) return fail(ctx, -1, "gguf upload: bad handle, tensor id or destination");
    if (dst_bytes < t->size)
        return fail(ctx, -1, "gguf upload: destination %llu < %llu bytes for %s", (unsigned long long)dst_bytes,
                        (unsigned long long)t->size, t->name.c_str());
    return upload_segments(ctx, g, *t, (uint8_t *)d_dst, t->size, 0);
}

int gpu_gguf_upload_f32(gpu_ctx_t *ctx, const gpu_gguf_t *g, int64_t id, float *d_dst, int64_t n) {
    if (!ctx) return -1;
    const fo::GgufTensor *t = tensor_at(g, id);
    if (!t || !d_dst) return fail(ctx, -1, "gguf upload_f32: bad handle, tensor id or destination");
    const int64_t ne = elements(*t);
    if (n != ne) return fail(ctx, -1, "gguf upload_f32: %s has %lld elements, not %lld", t->name.c_str(),
                                 (long long)ne, (long long)n);
    const int ty = t->type;
    if (ty == GGML_TYPE_F32) return upload_segments(ctx, g, *t, (uint8_t *)d_dst, t->size, 0);
    const int bv = fomoe_block_values(ty);
    if (bv == 0 || ne % bv)
        return fail(ctx, -1, "gguf upload_f32: %s: type %d has no fp32 conversion", t->name.c_str(), ty);
    // raw bytes into the context's staging buffer, then one conversion launch
    HIPC(ensure(ctx->staging, ctx->staging_cap, (size_t)t->size));
    const int rc = upload_segments(ctx, g, *t, ctx->staging, t->size, 0);
    if (rc) return rc;
    HIPC(fo::launch_dequant(ty, ctx->staging, d_dst, ne, ctx->stream));
    HIPC(hipStreamSynchronize(ctx->stream));
    return 0;
}

void gpu_gguf_free_moe_layer(gpu_ctx_t *ctx, gpu_moe_layer_t *L) {
    if (!ctx || !L) return;
    (void)hipStreamSynchronize(ctx->stream);
    const void *p[] = {L->router, L->experts, L->shared, L->shared_gate_vec, L->norm_w};
    for (const void *q : p)
        if (q) (void)hipFree(const_cast<void *>(q));
    L->router = nullptr;
    L->experts = nullptr;
    L->shared = nullptr;
    L->shared_gate_vec = nullptr;
    L->norm_w = nullptr;
}

int gpu_gguf_load_moe_layer(gpu_ctx_t *ctx, const gpu_gguf_t *g, int blk, gpu_moe_layer_t *L) {
    if (!ctx) return -1;
    if (!g || !L || blk < 0) return fail(ctx, -1, "gguf layer: bad arguments");
    auto find = [&](const char *what) -> const fo::GgufTensor * {
        char name[128];
        snprintf(name, sizeof name, "blk.%d.%s.weight", blk, what);
        return tensor_at(g, g->f.find_tensor(name));
    };
    const fo::GgufTensor *tg = find("ffn_gate_exps"), *tu = find("ffn_up_exps"), *td = find("ffn_down_exps"),
                         *tr = find("ffn_gate_inp");
    if (!tg || !tu || !td || !tr) return fail(ctx, -1, "gguf layer: block %d has no routed-expert tensors", blk);
    // ggml dims: gate/up [H, F, E], down [F, H, E], router [H, E]
    const int64_t H = tg->dims[0], F = tg->dims[1], E = tg->dims[2];
    if (tg->n_dims != 3 || tu->n_dims != 3 || td->n_dims != 3 || tu->dims[0] != H || tu->dims[1] != F ||
        tu->dims[2] != E || td->dims[0] != F || td->dims[1] != H || td->dims[2] != E || tr->dims[0] != H ||
        tr->dims[1] != E || H <= 0 || F <= 0 || E <= 0 || E > 1024 || H > INT32_MAX || F > INT32_MAX)
        return fail(ctx, -1, "gguf layer: block %d has inconsistent expert shapes", blk);
    if (!layer_type(tg->type) || !layer_type(tu->type) || !layer_type(td->type))
        return fail(ctx, -1, "gguf layer: block %d expert types %d/%d/%d unsupported", blk, tg->type, tu->type,
                        td->type);
    const uint64_t gs = fomoe_row_bytes(tg->type, H) * F, us = fomoe_row_bytes(tu->type, H) * F,
                   ds = fomoe_row_bytes(td->type, F) * H;
    if (gs == 0 || us == 0 || ds == 0 || tg->size != gs * E || tu->size != us * E || td->size != ds * E)
        return fail(ctx, -1, "gguf layer: block %d expert tensor sizes do not match their shapes", blk);
    const char *arch = gpu_gguf_get_str(g, "general.architecture");
    int64_t k = 0;
    double eps = 1e-6;
    if (arch) {
        const std::string a(arch);
        if (gpu_gguf_get_int(g, (a + ".expert_used_count").c_str(), &k) != 0) k = 0;
        (void)gpu_gguf_get_float(g, (a + ".attention.layer_norm_rms_epsilon").c_str(), &eps);
    }
    if (k <= 0 || k > 16 || k > E) return fail(ctx, -1, "gguf layer: expert_used_count %lld unusable", (long long)k);

    const fo::GgufTensor *sg = find("ffn_gate_shexp"), *su = find("ffn_up_shexp"), *sd = find("ffn_down_shexp"),
                         *sv = find("ffn_gate_inp_shexp"), *nw = find("post_attention_norm");
    if (!nw) nw = find("ffn_norm");
    const bool shared = sg && su && sd;
    uint64_t sgs = 0, sus = 0, sds = 0;
    int64_t Fs = 0;
    if (shared) {
        // ggml dims: gate/up [H, F_s], down [F_s, H], each in its own type
        // (reference src/model.c:164, 365-371)
        Fs = sg->dims[1];
        int64_t key_fs = 0;
        if (arch && gpu_gguf_get_int(g, (std::string(arch) + ".expert_shared_feed_forward_length").c_str(),
                                     &key_fs) == 0 && key_fs != Fs)
            return fail(ctx, -1, "gguf layer: block %d shared expert has %lld rows, the model key says %lld", blk,
                        (long long)Fs, (long long)key_fs);
        if (sg->n_dims != 2 || su->n_dims != 2 || sd->n_dims != 2 || sg->dims[0] != H || su->dims[0] != H ||
            su->dims[1] != Fs || sd->dims[0] != Fs || sd->dims[1] != H || Fs <= 0 || Fs > INT32_MAX ||
            !layer_type(sg->type) || !layer_type(su->type) || !layer_type(sd->type))
            return fail(ctx, -1, "gguf layer: block %d shared expert shape/type unsupported", blk);
        sgs = sg->size; sus = su->size; sds = sd->size;
        if (sgs != fomoe_row_bytes(sg->type, H) * Fs || sus != fomoe_row_bytes(su->type, H) * Fs ||
            sds != fomoe_row_bytes(sd->type, Fs) * H)
            return fail(ctx, -1, "gguf layer: block %d shared tensor sizes do not match their shapes", blk);
    }
    if (sv && elements(*sv) != H) return fail(ctx, -1, "gguf layer: block %d shared gate vector is not [H]", blk);
    if (nw && elements(*nw) != H) return fail(ctx, -1, "gguf layer: block %d norm weight is not [H]", blk);

    gpu_moe_layer_t out;
    memset(&out, 0, sizeof out);
    out.n_embd = (int)H;
    out.inter = (int)F;
    out.n_experts = (int)E;
    out.k = (int)k;
    out.gate_type = tg->type;
    out.up_type = tu->type;
    out.down_type = td->type;
    out.gate_size = gs;
    out.up_size = us;
    out.expert_stride = (gs + us + ds + kStoreAlign - 1) / kStoreAlign * kStoreAlign;
    out.shared_inter = (int)Fs;
    out.shared_gate_size = sgs;
    out.shared_up_size = sus;
    out.shared_gate_type = shared ? sg->type : 0;
    out.shared_up_type = shared ? su->type : 0;
    out.shared_down_type = shared ? sd->type : 0;
    out.eps = (float)eps;

    int rc = 0;
    auto alloc = [&](uint64_t bytes) -> void * {
        void *p = nullptr;
        if (rc == 0 && hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            rc = fail(ctx, -2, "gguf layer: hipMalloc(%llu) failed", (unsigned long long)bytes);
            p = nullptr;
        }
        return p;
    };
    uint8_t *ex = (uint8_t *)alloc((uint64_t)E * out.expert_stride);
    out.experts = ex;
    float *router = (float *)alloc((uint64_t)E * H * 4);
    out.router = router;
    uint8_t *sh = shared ? (uint8_t *)alloc(sgs + sus + sds) : nullptr;
    out.shared = sh;
    float *svec = sv ? (float *)alloc((uint64_t)H * 4) : nullptr;
    out.shared_gate_vec = svec;
    float *norm = nw ? (float *)alloc((uint64_t)H * 4) : nullptr;
    out.norm_w = norm;
    // the padding between an expert's down block and the next expert stays zero
    if (rc == 0 && out.expert_stride > gs + us + ds &&
        hipMemsetAsync(ex, 0, (uint64_t)E * out.expert_stride, ctx->stream) != hipSuccess)
        rc = fail(ctx, -2, "gguf layer: clearing the expert blobs failed");
    if (rc == 0) rc = upload_segments(ctx, g, *tg, ex, gs, out.expert_stride);
    if (rc == 0) rc = upload_segments(ctx, g, *tu, ex + gs, us, out.expert_stride);
    if (rc == 0) rc = upload_segments(ctx, g, *td, ex + gs + us, ds, out.expert_stride);
    if (rc == 0) rc = gpu_gguf_upload_f32(ctx, g, tr - g->f.tensors.data(), router, E * H);
    if (rc == 0 && shared) rc = upload_segments(ctx, g, *sg, sh, sgs, 0);
    if (rc == 0 && shared) rc = upload_segments(ctx, g, *su, sh + sgs, sus, 0);
    if (rc == 0 && shared) rc = upload_segments(ctx, g, *sd, sh + sgs + sus, sds, 0);
    if (rc == 0 && sv) rc = gpu_gguf_upload_f32(ctx, g, sv - g->f.tensors.data(), svec, H);
    if (rc == 0 && nw) rc = gpu_gguf_upload_f32(ctx, g, nw - g->f.tensors.data(), norm, H);
    if (rc != 0) {
        const std::string keep = ctx->err;
        gpu_gguf_free_moe_layer(ctx, &out);
        ctx->err = keep;
        return rc;
    }
    *L = out;
    return 0;
}

}  // extern "C"
