// libptmi runtime: device/stream lifetime, error reporting, the weight
// residency registry and the host-pointer pt_matvec_fn drop-in.
#include "ptmi_internal.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace ptmi {

namespace {

// A registered plain host buffer and its device copy (same layout).
struct HostBuffer {
    const char *host;
    size_t bytes;
    char *dev;
};

struct LibState {
    bool inited = false;
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<Resident *> residents;
    std::vector<HostBuffer> buffers;
    float *scratch[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t scratch_cap[4] = {0, 0, 0, 0};
    int status = PTMI_OK;
    char err[512] = {0};
};

LibState g;

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

int set_error(int status, const char *fmt, ...) {
    g.status = status;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g.err, sizeof(g.err), fmt, ap);
    va_end(ap);
    return status;
}

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return PTMI_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return set_error(PTMI_ERR_OOM, "%s: %s", what, hipGetErrorString(e));
    return set_error(PTMI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

static int init_device(int device) {
    if (g.inited) {
        if (device != g.device) return set_error(PTMI_ERR_STATE, "already initialised on device %d", g.device);
        return PTMI_OK;
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return set_error(PTMI_ERR_NODEV, "no HIP device visible");
    if (device < 0 || device >= count) return set_error(PTMI_ERR_ARG, "device %d out of range (%d)", device, count);
    PTMI_HIP(hipSetDevice(device));
    int st = gemm_scratch_setup(device);
    if (st) return st;
    PTMI_HIP(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
    g.device = device;
    g.inited = true;
    return PTMI_OK;
}

int ensure_init() { return g.inited ? PTMI_OK : init_device(0); }

hipStream_t lib_stream() { return g.stream; }
bool lib_initialised() { return g.inited; }
int lib_device() { return g.device; }

float *scratch_buf(int slot, size_t floats) {
    if (slot < 0 || slot >= 4) return nullptr;
    if (floats <= g.scratch_cap[slot]) return g.scratch[slot];
    if (g.scratch[slot]) {
        (void)hipStreamSynchronize(g.stream);
        (void)hipFree(g.scratch[slot]);
        g.scratch[slot] = nullptr;
        g.scratch_cap[slot] = 0;
    }
    size_t cap = align_up(floats, 1u << 16);
    float *p = nullptr;
    if (hipMalloc(&p, cap * sizeof(float)) != hipSuccess) {
        set_error(PTMI_ERR_OOM, "scratch allocation of %zu bytes failed", cap * sizeof(float));
        return nullptr;
    }
    g.scratch[slot] = p;
    g.scratch_cap[slot] = cap;
    return p;
}

// ── llama2.c header (pitorch/model/llama2.c:9-19, 21-47) ─────────────────
int parse_config(const void *blob, size_t bytes, Config *c) {
    if (!blob || bytes < 28) return set_error(PTMI_ERR_ARG, "blob too small for the 28-byte header");
    const int32_t *h = (const int32_t *)blob;
    c->dim = h[0]; c->hidden = h[1]; c->n_layers = h[2]; c->n_heads = h[3];
    c->n_kv_heads = h[4];
    c->shared = h[5] > 0;
    c->vocab = h[5] > 0 ? h[5] : -h[5];
    c->seq_len = h[6];
    if (c->dim <= 0 || c->hidden <= 0 || c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
        c->vocab <= 0 || c->seq_len <= 0 || c->dim % c->n_heads || c->n_heads % c->n_kv_heads)
        return set_error(PTMI_ERR_ARG, "bad llama2 header (%d %d %d %d %d %d %d)", h[0], h[1], h[2], h[3],
                         h[4], h[5], h[6]);
    c->head_dim = c->dim / c->n_heads;
    c->kv_dim = c->n_kv_heads * c->head_dim;
    return PTMI_OK;
}

static void host_offsets(Resident *r) {
    const Config &c = r->c;
    size_t D = c.dim, H = c.hidden, L = c.n_layers, KV = c.kv_dim, V = c.vocab;
    size_t o = 0;
    r->off_emb = o;       o += V * D;
    r->off_rms_att = o;   o += L * D;
    r->off_wq = o;        o += L * D * D;
    r->off_wk = o;        o += L * KV * D;
    r->off_wv = o;        o += L * KV * D;
    r->off_wo = o;        o += L * D * D;
    r->off_rms_ffn = o;   o += L * D;
    r->off_w1 = o;        o += L * H * D;
    r->off_w2 = o;        o += L * D * H;
    r->off_w3 = o;        o += L * H * D;
    r->off_rms_final = o; o += D;
    o += 2 * ((size_t)c.seq_len * c.head_dim / 2);     // freq_cis real, imag
    r->off_wcls = c.shared ? r->off_emb : o;
    if (!c.shared) o += V * D;
    r->off_end = o;
}

static HostBuffer *find_buffer(const void *p) {
    for (HostBuffer &b : g.buffers)
        if ((const char *)p >= b.host && (const char *)p < b.host + b.bytes) return &b;
    return nullptr;
}

Resident *find_resident(const void *p) {
    for (Resident *r : g.residents) {
        const char *lo = r->blob, *hi = r->blob + r->bytes;
        if ((const char *)p >= lo && (const char *)p < hi) return r;
    }
    return nullptr;
}

// Copy helpers for the device layout.
//   wqkv[l] = [wq_l ; wk_l ; wv_l]           rows D + 2*KV, cols D
//   w13[l]  = rows interleaved w1_l[i], w3_l[i]  rows 2H, cols D
static int copy_layout(Resident *r, hipStream_t s, bool to_device, void *hblob) {
    const Config &c = r->c;
    size_t D = c.dim, H = c.hidden, L = c.n_layers, KV = c.kv_dim, V = c.vocab;
    char *hb = (char *)hblob + 28;
    auto hp = [&](size_t off) { return (void *)(hb + off * sizeof(float)); };
    const size_t fs = sizeof(float);
    hipMemcpyKind kind = to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    // plain blocks
    struct Plain { float *dev; size_t off, n; };
    Plain plain[] = {{r->emb, r->off_emb, V * D}, {r->rms_att, r->off_rms_att, L * D},
                     {r->wo, r->off_wo, L * D * D}, {r->rms_ffn, r->off_rms_ffn, L * D},
                     {r->w2, r->off_w2, L * D * H}, {r->rms_final, r->off_rms_final, D}};
    for (auto &b : plain) {
        if (to_device) PTMI_HIP(hipMemcpyAsync(b.dev, hp(b.off), b.n * fs, kind, s));
        else PTMI_HIP(hipMemcpyAsync(hp(b.off), b.dev, b.n * fs, kind, s));
    }
    if (!c.shared) {
        if (to_device) PTMI_HIP(hipMemcpyAsync(r->wcls, hp(r->off_wcls), V * D * fs, kind, s));
        else PTMI_HIP(hipMemcpyAsync(hp(r->off_wcls), r->wcls, V * D * fs, kind, s));
    }
    // QKV: per layer, blocks of D*D / KV*D floats into rows of wqkv
    const size_t qkv_pitch = (D + 2 * KV) * D * fs;
    struct Strided { size_t dev_off, host_off, width; };
    Strided qkv[] = {{0, r->off_wq, D * D * fs}, {D * D, r->off_wk, KV * D * fs},
                     {(D + KV) * D, r->off_wv, KV * D * fs}};
    for (auto &b : qkv) {
        float *d = r->wqkv + b.dev_off;
        if (to_device) PTMI_HIP(hipMemcpy2DAsync(d, qkv_pitch, hp(b.host_off), b.width, b.width, L, kind, s));
        else PTMI_HIP(hipMemcpy2DAsync(hp(b.host_off), b.width, d, qkv_pitch, b.width, L, kind, s));
    }
    // w1 -> even rows, w3 -> odd rows of w13
    Strided ffn[] = {{0, r->off_w1, D * fs}, {D, r->off_w3, D * fs}};
    for (auto &b : ffn) {
        float *d = r->w13 + b.dev_off;
        if (to_device) PTMI_HIP(hipMemcpy2DAsync(d, 2 * D * fs, hp(b.host_off), D * fs, D * fs, L * H, kind, s));
        else PTMI_HIP(hipMemcpy2DAsync(hp(b.host_off), D * fs, d, 2 * D * fs, D * fs, L * H, kind, s));
    }
    return PTMI_OK;
}

int upload_resident(Resident *r, hipStream_t s) { return copy_layout(r, s, true, (void *)r->blob); }

int download_resident(Resident *r, void *blob, hipStream_t s) {
    int st = copy_layout(r, s, false, blob);
    if (st) return st;
    PTMI_HIP(hipStreamSynchronize(s));
    return PTMI_OK;
}

// A blob is looked up by its host address.  An existing registration is
// shared only when the size and the 28-byte header are the ones it was
// registered with; anything else at that address is an error (the caller
// must release the old registration first), so a new blob at a reused
// address never silently runs on another blob's device copy.
Resident *register_blob(const void *blob, size_t bytes, bool explicit_hold, int *status) {
    *status = ensure_init();
    if (*status) return nullptr;
    if (!blob || bytes < 28) {
        *status = set_error(PTMI_ERR_ARG, "blob too small for the 28-byte header");
        return nullptr;
    }
    if (Resident *r = find_resident(blob)) {
        if (r->blob != (const char *)blob) {
            *status = set_error(PTMI_ERR_ARG, "blob overlaps an already registered blob");
            return nullptr;
        }
        if (r->bytes != bytes || memcmp(r->header, blob, sizeof(r->header)) != 0) {
            *status = set_error(PTMI_ERR_STATE,
                                "a different blob (%zu bytes) is still registered at %p: release it first",
                                r->bytes, blob);
            return nullptr;
        }
        if (explicit_hold) r->explicit_holds++;
        else r->model_holds++;
        return r;
    }
    for (const HostBuffer &b : g.buffers)
        if ((const char *)blob < b.host + b.bytes && b.host < (const char *)blob + bytes) {
            *status = set_error(PTMI_ERR_ARG, "blob overlaps a registered buffer");
            return nullptr;
        }
    Resident *r = new Resident();
    r->blob = (const char *)blob;
    r->bytes = bytes;
    memcpy(r->header, blob, sizeof(r->header));
    r->explicit_holds = explicit_hold ? 1 : 0;
    r->model_holds = explicit_hold ? 0 : 1;
    if ((*status = parse_config(blob, bytes, &r->c))) { delete r; return nullptr; }
    host_offsets(r);
    if (28 + r->off_end * sizeof(float) > bytes) {
        *status = set_error(PTMI_ERR_ARG, "blob is %zu bytes, header needs %zu", bytes,
                            28 + r->off_end * sizeof(float));
        delete r;
        return nullptr;
    }
    const Config &c = r->c;
    size_t D = c.dim, H = c.hidden, L = c.n_layers, KV = c.kv_dim, V = c.vocab;
    const size_t al = 64;   // 256-byte alignment for every tensor
    size_t sizes[] = {V * D, L * D, L * (D + 2 * KV) * D, L * D * D, L * D, L * 2 * H * D, L * D * H, D,
                      c.shared ? 0 : V * D};
    size_t total = 0;
    for (size_t s : sizes) total += align_up(s, al);
    float *mem = nullptr;
    hipError_t e = hipMalloc(&mem, total * sizeof(float));
    if (e != hipSuccess) { *status = hip_check(e, "hipMalloc(weights)"); delete r; return nullptr; }
    r->mem = mem;
    r->mem_floats = total;
    float **dst[] = {&r->emb, &r->rms_att, &r->wqkv, &r->wo, &r->rms_ffn, &r->w13, &r->w2, &r->rms_final, &r->wcls};
    size_t o = 0;
    for (int i = 0; i < 9; i++) { *dst[i] = mem + o; o += align_up(sizes[i], al); }
    if (c.shared) r->wcls = r->emb;
    if ((*status = upload_resident(r, g.stream)) || (*status = hip_check(hipStreamSynchronize(g.stream), "upload"))) {
        (void)hipFree(mem);
        delete r;
        return nullptr;
    }
    g.residents.push_back(r);
    return r;
}

static void free_resident(Resident *r) {
    for (size_t i = 0; i < g.residents.size(); i++) {
        if (g.residents[i] == r) {
            g.residents.erase(g.residents.begin() + i);
            break;
        }
    }
    (void)hipStreamSynchronize(g.stream);
    (void)hipFree(r->mem);
    delete r;
}

void release_blob(Resident *r) {
    if (!r) return;
    if (r->model_holds > 0) r->model_holds--;
    if (r->model_holds == 0 && r->explicit_holds == 0) free_resident(r);
}

// Map a host pointer W (row start inside a registered tensor) to the device
// copy.  Returns false when W is not a whole-row view of one tensor block
// that is contiguous in the device layout.
static bool resolve(const Resident *r, const float *W, int out_dim, int in_dim, const float **dW, long *ld) {
    const float *base = (const float *)(r->blob + 28);
    if (W < base) return false;
    const size_t off = (size_t)(W - base);
    const Config &c = r->c;
    const size_t D = c.dim, H = c.hidden, L = c.n_layers, KV = c.kv_dim, V = c.vocab;
    struct T { size_t off, rows_per_layer, cols, layers; int kind; };
    // kind: 0 plain, 1 wq, 2 wk, 3 wv, 4 w1, 5 w3
    const T ts[] = {{r->off_emb, V, D, 1, 0},       {r->off_wq, D, D, L, 1},  {r->off_wk, KV, D, L, 2},
                    {r->off_wv, KV, D, L, 3},       {r->off_wo, D, D, L, 0},  {r->off_w1, H, D, L, 4},
                    {r->off_w2, D, H, L, 0},        {r->off_w3, H, D, L, 5},
                    {r->off_wcls, V, D, c.shared ? 0u : 1u, 0}};
    for (const T &t : ts) {
        const size_t n = t.rows_per_layer * t.cols * t.layers;
        if (n == 0 || off < t.off || off >= t.off + n) continue;
        if ((size_t)in_dim != t.cols) return false;
        const size_t lo = off - t.off;
        if (lo % t.cols) return false;
        const size_t row = lo / t.cols, layer = row / t.rows_per_layer, rl = row % t.rows_per_layer;
        if (rl + (size_t)out_dim > t.rows_per_layer) return false;   // crosses a layer block
        const float *dev = nullptr;
        long stride = (long)t.cols;
        switch (t.kind) {
        case 0: {
            const float *d0 = t.off == r->off_emb ? r->emb : t.off == r->off_wo ? r->wo
                            : t.off == r->off_w2 ? r->w2 : r->wcls;
            dev = d0 + row * t.cols;
            break;
        }
        case 1: dev = r->wqkv + (layer * (D + 2 * KV) + rl) * D; break;
        case 2: dev = r->wqkv + (layer * (D + 2 * KV) + D + rl) * D; break;
        case 3: dev = r->wqkv + (layer * (D + 2 * KV) + D + KV + rl) * D; break;
        case 4: dev = r->w13 + (layer * 2 * H + 2 * rl) * D; stride = 2 * (long)D; break;
        case 5: dev = r->w13 + (layer * 2 * H + 2 * rl + 1) * D; stride = 2 * (long)D; break;
        }
        *dW = dev;
        *ld = stride;
        return true;
    }
    return false;
}

}  // namespace ptmi

using namespace ptmi;

extern "C" {

int ptmi_init(int device) { return init_device(device); }

void ptmi_shutdown(void) {
    if (!g.inited) return;
    (void)hipStreamSynchronize(g.stream);
    for (Resident *r : g.residents) { (void)hipFree(r->mem); delete r; }
    g.residents.clear();
    for (HostBuffer &b : g.buffers) (void)hipFree(b.dev);
    g.buffers.clear();
    for (int i = 0; i < 4; i++) {
        if (g.scratch[i]) (void)hipFree(g.scratch[i]);
        g.scratch[i] = nullptr;
        g.scratch_cap[i] = 0;
    }
    (void)hipStreamDestroy(g.stream);
    g.stream = nullptr;
    g.inited = false;
}

const char *ptmi_last_error(void) { return g.err; }
int ptmi_last_status(void) { return g.status; }

void *ptmi_stream(void) {
    if (ensure_init()) return nullptr;
    return (void *)g.stream;
}

int ptmi_sync(void) {
    int st = ensure_init();
    if (st) return st;
    PTMI_HIP(hipStreamSynchronize(g.stream));
    return PTMI_OK;
}

int ptmi_register_weights(const void *blob, size_t bytes) {
    int st = PTMI_OK;
    register_blob(blob, bytes, true, &st);
    return st;
}

int ptmi_register_buffer(const void *p, size_t bytes) {
    int st = ensure_init();
    if (st) return st;
    if (!p || bytes == 0) return set_error(PTMI_ERR_ARG, "ptmi_register_buffer: empty buffer");
    const char *lo = (const char *)p, *hi = lo + bytes;
    for (const HostBuffer &b : g.buffers)
        if (lo < b.host + b.bytes && b.host < hi) return set_error(PTMI_ERR_ARG, "buffer %p overlaps a registered buffer", p);
    for (const Resident *r : g.residents)
        if (lo < r->blob + r->bytes && r->blob < hi) return set_error(PTMI_ERR_ARG, "buffer %p overlaps a registered blob", p);
    char *dev = nullptr;
    PTMI_HIP(hipMalloc(&dev, bytes));
    hipError_t e = hipMemcpyAsync(dev, p, bytes, hipMemcpyHostToDevice, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    if (e != hipSuccess) { (void)hipFree(dev); return hip_check(e, "ptmi_register_buffer upload"); }
    g.buffers.push_back(HostBuffer{lo, bytes, dev});
    return PTMI_OK;
}

int ptmi_unregister_buffer(const void *p) {
    for (size_t i = 0; i < g.buffers.size(); i++) {
        if (g.buffers[i].host != (const char *)p) continue;
        (void)hipStreamSynchronize(g.stream);
        (void)hipFree(g.buffers[i].dev);
        g.buffers.erase(g.buffers.begin() + (long)i);
        return PTMI_OK;
    }
    return set_error(PTMI_ERR_ARG, "buffer %p is not registered", p);
}

int ptmi_invalidate(const void *ptr, size_t bytes) {
    int st = ensure_init();
    if (st) return st;
    if (HostBuffer *b = find_buffer(ptr)) {      // re-upload the part written, clipped to the buffer
        const size_t off = (size_t)((const char *)ptr - b->host), n = std::min(bytes, b->bytes - off);
        PTMI_HIP(hipMemcpyAsync(b->dev + off, ptr, n, hipMemcpyHostToDevice, g.stream));
        PTMI_HIP(hipStreamSynchronize(g.stream));
        return PTMI_OK;
    }
    Resident *r = find_resident(ptr);
    if (!r) return PTMI_OK;            // not resident: nothing cached
    (void)bytes;                       // whole-tensor granularity: re-upload all
    if ((st = upload_resident(r, g.stream))) return st;
    PTMI_HIP(hipStreamSynchronize(g.stream));
    return PTMI_OK;
}

int ptmi_unregister_weights(const void *blob) {
    for (Resident *r : g.residents) {
        if (r->blob != (const char *)blob) continue;
        if (r->model_holds > 0)
            return set_error(PTMI_ERR_STATE, "blob %p is still used by %d model(s): destroy them first", blob,
                             r->model_holds);
        if (r->explicit_holds == 0)
            return set_error(PTMI_ERR_STATE, "blob %p has no ptmi_register_weights registration", blob);
        if (--r->explicit_holds == 0) free_resident(r);
        return PTMI_OK;
    }
    return set_error(PTMI_ERR_ARG, "blob %p is not registered", blob);
}

int ptmi_matvec_dev(const float *dW, long ld, const float *dx, float *dy, int out_dim, int in_dim,
                    void *stream) {
    int st = ensure_init();
    if (st) return st;
    MatvecParams p = {};
    p.W = dW; p.ld = ld; p.rows = out_dim; p.n = in_dim; p.x = dx; p.y = dy;
    p.pro = PRO_NONE; p.epi = EPI_STORE;
    return launch_matvec(p, stream ? (hipStream_t)stream : g.stream);
}

int ptmi_matvec_dev_xreread(const float *dW, long ld, const float *dx, float *dy, int out_dim, int in_dim,
                            void *stream) {
    int st = ensure_init();
    if (st) return st;
    MatvecParams p = {};
    p.W = dW; p.ld = ld; p.rows = out_dim; p.n = in_dim; p.x = dx; p.y = dy;
    p.pro = PRO_NONE; p.epi = EPI_STORE;
    return launch_matvec(p, stream ? (hipStream_t)stream : g.stream, nullptr, nullptr, true);
}

int ptmi_matvec_checked(const float *W, const float *x, float *y, int out_dim, int in_dim) {
    int st = ensure_init();
    if (st) return st;
    if (!W || !x || !y || out_dim <= 0 || in_dim <= 0)
        return set_error(PTMI_ERR_ARG, "ptmi_matvec: bad arguments (out=%d in=%d)", out_dim, in_dim);
    hipStream_t s = g.stream;
    const float *dW = nullptr;
    long ld = in_dim;
    Resident *r = find_resident(W);
    const HostBuffer *hb = r ? nullptr : find_buffer(W);
    const size_t w_bytes = (size_t)out_dim * in_dim * sizeof(float);
    if (hb && (size_t)((const char *)W - hb->host) + w_bytes <= hb->bytes) {
        // inside a registered plain buffer: its device copy
        dW = reinterpret_cast<const float *>(hb->dev + ((const char *)W - hb->host));
    } else if (!(r && resolve(r, W, out_dim, in_dim, &dW, &ld))) {
        // Not a resident tensor view (e.g. an unregistered host-transposed
        // scratch copy): upload for this call.
        float *w = scratch_buf(0, (size_t)out_dim * in_dim);
        if (!w) return g.status;
        PTMI_HIP(hipMemcpyAsync(w, W, (size_t)out_dim * in_dim * sizeof(float), hipMemcpyHostToDevice, s));
        dW = w;
        ld = in_dim;
    }
    float *dx = scratch_buf(1, (size_t)in_dim);
    float *dy = scratch_buf(2, (size_t)out_dim);
    if (!dx || !dy) return g.status;
    PTMI_HIP(hipMemcpyAsync(dx, x, (size_t)in_dim * sizeof(float), hipMemcpyHostToDevice, s));
    if ((st = ptmi_matvec_dev(dW, ld, dx, dy, out_dim, in_dim, s))) return st;
    PTMI_HIP(hipMemcpyAsync(y, dy, (size_t)out_dim * sizeof(float), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    return PTMI_OK;
}

void ptmi_matvec(const float *W, const float *x, float *y, int out_dim, int in_dim) {
    if (ptmi_matvec_checked(W, x, y, out_dim, in_dim) != PTMI_OK) {
        fprintf(stderr, "ptmi_matvec: %s\n", g.err);
        abort();
    }
}

}  // extern "C"
