// C ABI of the MoE block (include/qe_moe.h): context, flat expert arena,
// per-layer dense weights, scratch, and the forward entry points.
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/qe_moe.h"
#include "qe_kernels.h"

static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
#define HIP_TRY(expr)                                                                             \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) return fail(QE_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));    \
    } while (0)

struct qe_moe_ctx {
    int device = 0, n_layers = 0, t_max = 0;
    uint8_t *arena = nullptr;    // n_layers * 256 * EXPERT_BYTES
    float *router = nullptr;     // n_layers * 257 * 2048
    float *bias = nullptr;       // n_layers * 256
    uint8_t *sh_gu = nullptr;    // n_layers * SH_GU_BYTES
    uint8_t *sh_dn = nullptr;    // n_layers * SH_DN_BYTES
    float *post_norm = nullptr;  // n_layers * 2048
    std::vector<uint8_t> has_bias;
    std::vector<uint32_t> have;                  // per layer: HAVE_* bits of the tensors set so far
    std::vector<std::vector<uint8_t>> have_exp;  // per layer: which of the 256 experts were supplied
    QeScratch S{};
    QeProf prof;
    uint8_t *bias_on = nullptr;  // device copy of has_bias
    uint64_t *ex = nullptr;      // decode exchange words
    unsigned *sync = nullptr;    // decode launch epoch + exit counter
    unsigned *err_host = nullptr; // pinned, host-mapped: 0, or 1 + epoch of the last decode launch whose poll timed out
    unsigned *err_dev = nullptr;  // the same word as the kernels address it
    unsigned err_seen = 0;        // the value last reported
    unsigned prefill_seq = 0;     // prefill calls so far: a timed-out wait of one stores 0x80000000 | its number
    int spin_cap = QE_DECODE_SPIN_CAP;
    float *pingpong[2] = {nullptr, nullptr};
    std::vector<void *> allocs;
};

static int dalloc(qe_moe_ctx *c, void **p, size_t bytes, bool zero = true) {
    if (hipMalloc(p, bytes) != hipSuccess) {
        *p = nullptr;
        return fail(QE_ERR_OOM, "hipMalloc(%zu) failed", bytes);
    }
    c->allocs.push_back(*p);
    // scratch starts as zeros: the padding rows of the prefill tiles are read
    // (never stored), and must hold finite values
    if (zero && hipMemset(*p, 0, bytes) != hipSuccess) return fail(QE_ERR_HIP, "hipMemset(%zu) failed", bytes);
    return QE_OK;
}

static void free_all(qe_moe_ctx *c) {
    for (void *p : c->allocs) (void)hipFree(p);
    c->allocs.clear();
    if (c->err_host) (void)hipHostFree(c->err_host);
    c->err_host = nullptr;
}

// What a layer needs before a forward call may run on it.
enum : uint32_t { HAVE_NORM = 1, HAVE_ROUTER = 2, HAVE_SH_GU = 4, HAVE_SH_DN = 8, HAVE_ALL_DENSE = 15 };
static void mark_experts(qe_moe_ctx *c, int layer, int first, int n) {
    for (int e = first; e < first + n; ++e) c->have_exp[layer][e] = 1;
}
static bool layer_ready(const qe_moe_ctx *c, int layer, std::string &missing) {
    static const char *const names[4] = {"post_norm", "router", "sh_gu", "sh_down"};
    missing.clear();
    for (int b = 0; b < 4; ++b)
        if (!(c->have[layer] & (1u << b))) missing += std::string(missing.empty() ? "" : ", ") + names[b];
    int nexp = 0;
    for (uint8_t h : c->have_exp[layer]) nexp += h;
    if (nexp < QE_N_EXPERT)
        missing += std::string(missing.empty() ? "" : ", ") + std::to_string(QE_N_EXPERT - nexp) + " experts";
    return missing.empty();
}

// A decode launch whose exchange poll timed out leaves 1 + its epoch in the
// host-mapped error word.  Every poll that gives up writes it, and such writes
// to host memory can land after the host last looked, so the word is never
// cleared: each value is reported once, by the next call that looks.
static int take_decode_error(qe_moe_ctx *c, const char *where) {
    const unsigned v = __atomic_load_n(c->err_host, __ATOMIC_ACQUIRE);
    if (!v || v == c->err_seen) return QE_OK;
    c->err_seen = v;
    if (v & 0x80000000u)
        return fail(QE_ERR_STATE, "%s: prefill call %u timed out waiting for its gate/up workgroups; its outputs are invalid",
                    where, v & 0x7fffffffu);
    return fail(QE_ERR_STATE, "%s: the decode launch of epoch %u timed out waiting for an exchange; its outputs are invalid",
                where, v - 1u);
}

static QeLayerPtrs layer_ptrs(const qe_moe_ctx *c, int l) {
    QeLayerPtrs L;
    L.arena = c->arena + (size_t)l * QE_LAYER_EXPERT_BYTES;
    L.router = c->router + (size_t)l * QE_ROUTER_ROWS * QE_D;
    L.bias = c->has_bias[l] ? c->bias + (size_t)l * QE_N_EXPERT : nullptr;
    L.sh_gu = c->sh_gu + (size_t)l * QE_SH_GU_BYTES;
    L.sh_dn = c->sh_dn + (size_t)l * QE_SH_DN_BYTES;
    L.post_norm = c->post_norm + (size_t)l * QE_D;
    return L;
}

extern "C" {

const char *qe_moe_last_error(void) { return g_err.c_str(); }

size_t qe_moe_expert_bytes(void) { return QE_EXPERT_BYTES; }

int qe_moe_create(int device, int n_layers, int t_max, qe_moe_ctx **out) {
    if (!out || n_layers <= 0 || n_layers > 4096 || t_max <= 0 || t_max > QE_MOE_T_MAX)
        return fail(QE_ERR_ARG, "qe_moe_create: bad argument (n_layers=%d t_max=%d)", n_layers, t_max);
    *out = nullptr;
    HIP_TRY(hipSetDevice(device));
    qe_moe_ctx *c = new qe_moe_ctx();
    c->device = device;
    c->n_layers = n_layers;
    c->t_max = t_max;
    c->has_bias.assign(n_layers, 0);
    c->have.assign(n_layers, 0u);
    c->have_exp.assign(n_layers, std::vector<uint8_t>(QE_N_EXPERT, 0));
    const size_t L = (size_t)n_layers, T = (size_t)t_max, NP = T * QE_K_USED, T32 = (T + 31) & ~(size_t)31;
    const size_t max_items = NP / (QE_MFMA_MC / 2 + 1) + 1 + QE_N_EXPERT; // big items hold > MC / 2 pairs
    const size_t nch = (NP + 1023) / 1024;
    int rc = QE_OK;
    QeScratch &S = c->S;
#define A(ptr, bytes) \
    if (rc == QE_OK) rc = dalloc(c, (void **)&(ptr), (bytes))
    if (rc == QE_OK) rc = dalloc(c, (void **)&c->arena, L * QE_LAYER_EXPERT_BYTES, false); // written by upload/synth
    A(c->router, L * QE_ROUTER_BYTES);
    A(c->bias, L * QE_N_EXPERT * 4);
    A(c->sh_gu, L * QE_SH_GU_BYTES);
    A(c->sh_dn, L * QE_SH_DN_BYTES);
    A(c->post_norm, L * QE_D * 4);
    A(S.xn, T * QE_D * 4);
    A(S.xqp, T * QE_D);
    A(S.xs, T * (QE_D / 32) * 4);
    A(S.xhl, T32 * QE_D * 4);
    A(S.logits, T * QE_ROUTER_ROWS * 4);
    A(S.shgu, T32 * QE_FF_SH * 4);
    A(S.rpart, 8 * T * QE_N_EXPERT * 4);
    A(S.ids, NP * 4);
    A(S.wts, NP * 4);
    A(S.shg, T * 4);
    A(S.off, (QE_N_EXPERT + 1) * 4);
    A(S.pairs, NP * 4);
    A(S.items, max_items * sizeof(int4));
    A(S.n_items, 8);
    A(S.hqp, NP * QE_FF_EXP);
    A(S.hs, NP * (QE_FF_EXP / 32) * 4);
    A(S.sd, T * QE_D * 4);
    A(S.yp, NP * QE_D * 4);
    A(S.chunk_hist, nch * QE_N_EXPERT * 4);
    A(S.item_done, max_items * 4);
    A(c->bias_on, L);
    A(c->ex, (size_t)QE_DECODE_EX_WORDS * 8);
    A(c->sync, QE_DECODE_SYNC_WORDS * 4);
    A(c->pingpong[0], T * QE_D * 4);
    A(c->pingpong[1], T * QE_D * 4);
#undef A
    if (rc != QE_OK) {
        free_all(c);
        delete c;
        return rc;
    }
    if (rc == QE_OK) {
        void *h = nullptr, *d = nullptr;
        if (hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
            rc = fail(QE_ERR_OOM, "hipHostMalloc of the error word failed");
        else if ((c->err_host = (unsigned *)h), hipHostGetDevicePointer(&d, h, 0) != hipSuccess)
            rc = fail(QE_ERR_HIP, "hipHostGetDevicePointer of the error word failed");
        else {
            c->err_dev = (unsigned *)d;
            memset(h, 0, 256);
            S.err = c->err_dev;
        }
    }
    if (rc != QE_OK) {
        free_all(c);
        delete c;
        return rc;
    }
    S.t_max = t_max;
    S.prof = &c->prof;
    S.spin_cap = c->spin_cap;
    if (hipMemset(c->bias, 0, L * QE_N_EXPERT * 4) != hipSuccess ||
        hipMemset(c->bias_on, 0, L) != hipSuccess || hipMemset(c->sync, 0, QE_DECODE_SYNC_WORDS * 4) != hipSuccess ||
        hipMemset(c->ex, 0, (size_t)QE_DECODE_EX_WORDS * 8) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        free_all(c);
        delete c;
        return fail(QE_ERR_HIP, "qe_moe_create: initial memset failed");
    }
    if (qe_noalloc_prepare(nullptr) != hipSuccess) { // the no-allocation dispatch's scratch, looked up before any capture
        free_all(c);
        delete c;
        return fail(QE_ERR_HIP, "qe_moe_create: lookup of the static dispatch scratch failed");
    }
    *out = c;
    return QE_OK;
}

int qe_moe_destroy(qe_moe_ctx *c) {
    if (!c) return QE_OK;
    (void)hipSetDevice(c->device);
    (void)hipDeviceSynchronize();
    for (int i = 0; i < 2 * c->prof.cap; ++i) (void)hipEventDestroy(c->prof.ev[i]);
    delete[] c->prof.ev;
    delete[] c->prof.kid;
    free_all(c);
    delete c;
    return QE_OK;
}

int qe_moe_upload_experts(qe_moe_ctx *c, int layer, int first, int n, const void *src, int on_dev, void *stream) {
    if (!c || !src || layer < 0 || layer >= c->n_layers || first < 0 || n <= 0 || first + n > QE_N_EXPERT)
        return fail(QE_ERR_ARG, "qe_moe_upload_experts: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    uint8_t *dst = c->arena + (size_t)layer * QE_LAYER_EXPERT_BYTES + (size_t)first * QE_EXPERT_BYTES;
    HIP_TRY(hipMemcpyAsync(dst, src, (size_t)n * QE_EXPERT_BYTES, on_dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                           (hipStream_t)stream));
    if (!on_dev) HIP_TRY(hipStreamSynchronize((hipStream_t)stream)); /* host sources need not outlive the call */
    mark_experts(c, layer, first, n);
    return QE_OK;
}

int qe_moe_set_dense(qe_moe_ctx *c, int layer, const float *post_norm, const float *router, const float *bias,
                     const void *sh_gu, const void *sh_down, int on_dev, void *stream) {
    if (!c || layer < 0 || layer >= c->n_layers) return fail(QE_ERR_ARG, "qe_moe_set_dense: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    const hipMemcpyKind k = on_dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    hipStream_t s = (hipStream_t)stream;
    const QeLayerPtrs L = layer_ptrs(c, layer);
    // a tensor being replaced counts as missing until its copy has gone through:
    // a failed copy leaves the layer refused (QE_ERR_STATE), not running on
    // half-written weights
    const unsigned bits = (post_norm ? HAVE_NORM : 0u) | (router ? HAVE_ROUTER : 0u) | (sh_gu ? HAVE_SH_GU : 0u) |
                          (sh_down ? HAVE_SH_DN : 0u);
    c->have[layer] &= ~bits;
    if (post_norm) HIP_TRY(hipMemcpyAsync((void *)L.post_norm, post_norm, QE_D * 4, k, s));
    if (router) HIP_TRY(hipMemcpyAsync((void *)L.router, router, QE_ROUTER_BYTES, k, s));
    if (bias) {
        HIP_TRY(hipMemcpyAsync(c->bias + (size_t)layer * QE_N_EXPERT, bias, QE_N_EXPERT * 4, k, s));
        c->has_bias[layer] = 1;
        HIP_TRY(hipMemcpyAsync(c->bias_on + layer, &c->has_bias[layer], 1, hipMemcpyHostToDevice, s));
    }
    if (sh_gu) HIP_TRY(hipMemcpyAsync((void *)L.sh_gu, sh_gu, QE_SH_GU_BYTES, k, s));
    if (sh_down) HIP_TRY(hipMemcpyAsync((void *)L.sh_dn, sh_down, QE_SH_DN_BYTES, k, s));
    if (!on_dev) HIP_TRY(hipStreamSynchronize(s)); /* host sources need not outlive the call */
    c->have[layer] |= bits;
    return QE_OK;
}

// ---------------------------------------------------------------------------
// Pack-file loader.  File layout as engine/pack.h:45-54 (header "QE36PK01",
// entry table of {name[96], fmt, rows, cols, n, off, bytes}); the MoE tensors
// of layer N under the names Engine::Engine uploads (engine/qe.cpp:1051-1057):
// blk.N.post_norm (F32), blk.N.router + blk.N.sh_gate (F32, appended as router
// row 256), blk.N.sh_gate_proj + blk.N.sh_up (Q8, gate rows then up rows),
// blk.N.sh_down (Q8), and blk.N.experts (256 NL4 blobs, engine/qe.cpp:1177).
// Where the reference exits (engine/qe.cpp:57-67), this returns QE_ERR_ARG.
// ---------------------------------------------------------------------------
namespace {
struct PackHeaderRaw {
    char magic[8];
    uint32_t n_entries, pad;
    uint64_t table_off;
};
struct PackEntryRaw {
    char name[96];
    uint32_t fmt, rows, cols, n;
    uint64_t off, bytes;
};
static_assert(sizeof(PackHeaderRaw) == 24 && sizeof(PackEntryRaw) == 128, "pack layout of engine/pack.h");
enum { PK_F32 = 0, PK_Q8 = 1, PK_Q6 = 2, PK_NL4 = 3 };
struct MappedFile {
    uint8_t *base = nullptr;
    size_t size = 0;
    ~MappedFile() {
        if (base) munmap(base, size);
    }
};
}  // namespace

int qe_moe_load_pack(qe_moe_ctx *c, const char *path, int pack_first, int first_layer, int n_layers, void *stream) {
    if (!c || !path || pack_first < 0 || first_layer < 0 || n_layers <= 0 || first_layer + n_layers > c->n_layers)
        return fail(QE_ERR_ARG, "qe_moe_load_pack: bad argument");
    MappedFile f;
    {
        const int fd = open(path, O_RDONLY);
        if (fd < 0) return fail(QE_ERR_ARG, "qe_moe_load_pack: cannot open %s", path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size < (off_t)sizeof(PackHeaderRaw)) {
            close(fd);
            return fail(QE_ERR_ARG, "qe_moe_load_pack: %s is not a pack", path);
        }
        f.size = (size_t)st.st_size;
        void *m = mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (m == MAP_FAILED) return fail(QE_ERR_ARG, "qe_moe_load_pack: cannot map %s", path);
        f.base = (uint8_t *)m;
    }
    PackHeaderRaw h;
    memcpy(&h, f.base, sizeof h);
    if (memcmp(h.magic, "QE36PK01", 8) != 0) return fail(QE_ERR_ARG, "qe_moe_load_pack: bad magic in %s", path);
    if (h.table_off > f.size || (f.size - h.table_off) / sizeof(PackEntryRaw) < h.n_entries)
        return fail(QE_ERR_ARG, "qe_moe_load_pack: entry table past the end of %s", path);
    std::map<std::string, PackEntryRaw> ents;
    for (uint32_t i = 0; i < h.n_entries; ++i) {
        PackEntryRaw e;
        memcpy(&e, f.base + h.table_off + (size_t)i * sizeof e, sizeof e);
        e.name[sizeof e.name - 1] = 0;
        if (e.off > f.size || e.bytes > f.size - e.off)
            return fail(QE_ERR_ARG, "qe_moe_load_pack: entry %s past the end of the file", e.name);
        ents[e.name] = e;
    }
    // one tensor by name, checked for format, size and (for experts) count
    auto get = [&](const std::string &name, uint32_t fmt, size_t bytes, uint32_t n, const uint8_t **out) -> int {
        auto it = ents.find(name);
        if (it == ents.end()) return fail(QE_ERR_ARG, "qe_moe_load_pack: missing %s", name.c_str());
        const PackEntryRaw &e = it->second;
        if (e.fmt != fmt)
            return fail(QE_ERR_ARG, "qe_moe_load_pack: %s has format %u, this build takes %u", name.c_str(), e.fmt, fmt);
        if (e.bytes != bytes || e.n != n)
            return fail(QE_ERR_ARG, "qe_moe_load_pack: %s holds %llu bytes (n = %u), expected %zu (n = %u)", name.c_str(),
                        (unsigned long long)e.bytes, e.n, bytes, n);
        *out = f.base + e.off;
        return QE_OK;
    };
    HIP_TRY(hipSetDevice(c->device));
    hipStream_t s = (hipStream_t)stream;
    const hipMemcpyKind k = hipMemcpyHostToDevice;
    for (int i = 0; i < n_layers; ++i) {
        const int l = first_layer + i;
        const std::string pre = "blk." + std::to_string(pack_first + i) + ".";
        const uint8_t *pn, *rt, *sg, *gp, *up, *dn, *ex;
        int rc;
        if ((rc = get(pre + "post_norm", PK_F32, QE_D * 4, 1, &pn)) != QE_OK) return rc;
        if ((rc = get(pre + "router", PK_F32, (size_t)QE_N_EXPERT * QE_D * 4, 1, &rt)) != QE_OK) return rc;
        if ((rc = get(pre + "sh_gate", PK_F32, QE_D * 4, 1, &sg)) != QE_OK) return rc;
        if ((rc = get(pre + "sh_gate_proj", PK_Q8, QE_SH_GU_BYTES / 2, 1, &gp)) != QE_OK) return rc;
        if ((rc = get(pre + "sh_up", PK_Q8, QE_SH_GU_BYTES / 2, 1, &up)) != QE_OK) return rc;
        if ((rc = get(pre + "sh_down", PK_Q8, QE_SH_DN_BYTES, 1, &dn)) != QE_OK) return rc;
        if ((rc = get(pre + "experts", PK_NL4, QE_LAYER_EXPERT_BYTES, QE_N_EXPERT, &ex)) != QE_OK) return rc;
        const QeLayerPtrs L = layer_ptrs(c, l);
        HIP_TRY(hipMemcpyAsync(c->arena + (size_t)l * QE_LAYER_EXPERT_BYTES, ex, QE_LAYER_EXPERT_BYTES, k, s));
        HIP_TRY(hipMemcpyAsync((void *)L.post_norm, pn, QE_D * 4, k, s));
        HIP_TRY(hipMemcpyAsync((void *)L.router, rt, (size_t)QE_N_EXPERT * QE_D * 4, k, s));
        HIP_TRY(hipMemcpyAsync((void *)(L.router + (size_t)QE_N_EXPERT * QE_D), sg, QE_D * 4, k, s));
        HIP_TRY(hipMemcpyAsync((void *)L.sh_gu, gp, QE_SH_GU_BYTES / 2, k, s));
        HIP_TRY(hipMemcpyAsync((void *)(L.sh_gu + QE_SH_GU_BYTES / 2), up, QE_SH_GU_BYTES / 2, k, s));
        HIP_TRY(hipMemcpyAsync((void *)L.sh_dn, dn, QE_SH_DN_BYTES, k, s));
        c->has_bias[l] = 0;
        HIP_TRY(hipMemcpyAsync(c->bias_on + l, &c->has_bias[l], 1, hipMemcpyHostToDevice, s));
        HIP_TRY(hipStreamSynchronize(s)); // the mapping goes away with this call
        c->have[l] = HAVE_ALL_DENSE;
        mark_experts(c, l, 0, QE_N_EXPERT);
    }
    return QE_OK;
}

static int check_fwd(qe_moe_ctx *c, int layer, const void *in, const void *out, int T) {
    if (!c || !in || !out || T <= 0) return fail(QE_ERR_ARG, "forward: bad argument");
    if (layer < 0 || layer >= c->n_layers) return fail(QE_ERR_ARG, "forward: layer %d out of range", layer);
    if (T > c->t_max) return fail(QE_ERR_ARG, "forward: T=%d exceeds t_max=%d", T, c->t_max);
    std::string missing;
    if (!layer_ready(c, layer, missing)) return fail(QE_ERR_STATE, "forward: layer %d lacks %s", layer, missing.c_str());
    if (in == out) return fail(QE_ERR_ARG, "forward: output may not alias the input");
    return take_decode_error(c, "forward");
}

// T <= QE_SMALL_T: every layer of the range in one persistent launch.
static hipError_t run_decode(qe_moe_ctx *c, int first, int n, const float *in, float *out, int T, bool norm_res,
                             hipStream_t st, const float *exit_norm = nullptr, float *exit_xn = nullptr) {
    QeDecodeArgs d{};
    d.arena = c->arena; d.router = c->router; d.bias = c->bias; d.bias_on = c->bias_on;
    d.sh_gu = c->sh_gu; d.sh_dn = c->sh_dn; d.post_norm = c->post_norm;
    d.first_layer = first; d.n_layers = n; d.T = T; d.norm = norm_res; d.residual = norm_res;
    d.x_in = in; d.x_out = out;
    d.ex = c->ex;
    d.logits = c->S.logits; d.ids = c->S.ids; d.wts = c->S.wts; d.shg = c->S.shg; d.off = c->S.off; d.pairs = c->S.pairs;
    d.sd_out = c->S.sd; d.xn_out = c->S.xn;
    d.sync = c->sync; d.err = c->err_dev; d.spin_cap = c->spin_cap;
    d.exit_norm = exit_norm; d.exit_xn = exit_xn;
    ProfScope ps(&c->prof, QP_DECODE, st);
    return qe_launch_decode(d, st);
}

int qe_moe_forward(qe_moe_ctx *c, int layer, const float *x2, float *x, int T, void *stream) {
    int rc = check_fwd(c, layer, x2, x, T);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(c->device));
    if (T <= QE_SMALL_T) HIP_TRY(run_decode(c, layer, 1, x2, x, T, true, (hipStream_t)stream));
    else {
        c->S.err_val = 0x80000000u | (++c->prefill_seq & 0x7fffffffu);
        HIP_TRY(qe_launch_layer(layer_ptrs(c, layer), c->S, x2, true, x2, x, T, (hipStream_t)stream));
    }
    return QE_OK;
}

int qe_moe_forward_norm(qe_moe_ctx *c, int layer, const float *x2, float *x, int T, const float *next_norm, float *xn,
                        void *stream) {
    int rc = check_fwd(c, layer, x2, x, T);
    if (rc) return rc;
    if (!next_norm || !xn) return fail(QE_ERR_ARG, "forward_norm: next_norm and xn are required");
    if (xn == x || xn == x2) return fail(QE_ERR_ARG, "forward_norm: xn may not alias x or x2");
    HIP_TRY(hipSetDevice(c->device));
    if (T <= QE_SMALL_T)
        HIP_TRY(run_decode(c, layer, 1, x2, x, T, true, (hipStream_t)stream, next_norm, xn));
    else {
        c->S.err_val = 0x80000000u | (++c->prefill_seq & 0x7fffffffu);
        HIP_TRY(qe_launch_layer(layer_ptrs(c, layer), c->S, x2, true, x2, x, T, (hipStream_t)stream, next_norm, xn));
    }
    return QE_OK;
}

int qe_moe_forward_normed(qe_moe_ctx *c, int layer, const float *xn, float *y, int T, void *stream) {
    int rc = check_fwd(c, layer, xn, y, T);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(c->device));
    if (T <= QE_SMALL_T) HIP_TRY(run_decode(c, layer, 1, xn, y, T, false, (hipStream_t)stream));
    else {
        c->S.err_val = 0x80000000u | (++c->prefill_seq & 0x7fffffffu);
        HIP_TRY(qe_launch_layer(layer_ptrs(c, layer), c->S, xn, false, nullptr, y, T, (hipStream_t)stream));
    }
    return QE_OK;
}

int qe_moe_forward_stack(qe_moe_ctx *c, int first, int n, const float *x_in, float *x_out, int T, void *stream) {
    if (!c || n <= 0 || first < 0 || first + n > c->n_layers)
        return fail(QE_ERR_ARG, "forward_stack: bad layer range");
    if (x_in == x_out) return fail(QE_ERR_ARG, "forward_stack: output may not alias the input");
    if (T > 0 && T <= QE_SMALL_T) {
        for (int i = 0; i < n; ++i) {
            int rc = check_fwd(c, first + i, x_in, x_out, T);
            if (rc) return rc;
        }
        HIP_TRY(hipSetDevice(c->device));
        HIP_TRY(run_decode(c, first, n, x_in, x_out, T, true, (hipStream_t)stream));
        return QE_OK;
    }
    const float *cur = x_in;
    for (int i = 0; i < n; ++i) {
        float *dst = (i == n - 1) ? x_out : c->pingpong[i & 1];
        int rc = qe_moe_forward(c, first + i, cur, dst, T, stream);
        if (rc) return rc;
        cur = dst;
    }
    return QE_OK;
}

int qe_moe_get_routing(qe_moe_ctx *c, int T, int32_t *ids, float *wts, float *shg, int32_t *off, int32_t *pairs,
                       float *shared_out, void *stream) {
    if (!c || T <= 0 || T > c->t_max) return fail(QE_ERR_ARG, "get_routing: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    hipStream_t s = (hipStream_t)stream;
    const size_t np = (size_t)T * QE_K_USED;
    if (ids) HIP_TRY(hipMemcpyAsync(ids, c->S.ids, np * 4, hipMemcpyDeviceToHost, s));
    if (wts) HIP_TRY(hipMemcpyAsync(wts, c->S.wts, np * 4, hipMemcpyDeviceToHost, s));
    if (shg) HIP_TRY(hipMemcpyAsync(shg, c->S.shg, (size_t)T * 4, hipMemcpyDeviceToHost, s));
    if (off) HIP_TRY(hipMemcpyAsync(off, c->S.off, (QE_N_EXPERT + 1) * 4, hipMemcpyDeviceToHost, s));
    if (pairs) HIP_TRY(hipMemcpyAsync(pairs, c->S.pairs, np * 4, hipMemcpyDeviceToHost, s));
    if (shared_out) HIP_TRY(hipMemcpyAsync(shared_out, c->S.sd, (size_t)T * QE_D * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return take_decode_error(c, "get_routing");
}

int qe_moe_dispatch(qe_moe_ctx *c, const int32_t *ids, int T, void *stream) {
    if (!c || !ids || T <= 0 || T > c->t_max) return fail(QE_ERR_ARG, "dispatch: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpyAsync(c->S.ids, ids, (size_t)T * QE_K_USED * 4, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    HIP_TRY(qe_launch_dispatch(c->S, T, (hipStream_t)stream));
    return QE_OK;
}

int qe_moe_dispatch_noalloc(const int32_t *ids, int T, int32_t *off, int32_t *pairs, void *stream) {
    if (!ids || !off || !pairs) return fail(QE_ERR_ARG, "dispatch_noalloc: null pointer");
    if (T < 1 || T > QE_MOE_DISPATCH_NOALLOC_T_MAX)
        return fail(QE_ERR_ARG, "dispatch_noalloc: T=%d outside 1..%d (the static scratch's size)", T,
                    QE_MOE_DISPATCH_NOALLOC_T_MAX);
    HIP_TRY(qe_launch_dispatch_noalloc(ids, T, off, pairs, (hipStream_t)stream));
    return QE_OK;
}
static_assert(QE_MOE_DISPATCH_NOALLOC_T_MAX == QE_DISPATCH_NOALLOC_T_MAX, "header and library limits agree");
static_assert(QE_MOE_T_MAX == QE_LAYER_T_MAX, "header and library limits agree");

int qe_moe_get_logits(qe_moe_ctx *c, int T, float *logits, void *stream) {
    if (!c || !logits || T <= 0 || T > c->t_max) return fail(QE_ERR_ARG, "get_logits: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpyAsync(logits, c->S.logits, (size_t)T * QE_ROUTER_ROWS * 4, hipMemcpyDeviceToHost, (hipStream_t)stream));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return take_decode_error(c, "get_logits");
}

int qe_moe_check(qe_moe_ctx *c, void *stream) {
    if (!c) return fail(QE_ERR_ARG, "check: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return take_decode_error(c, "check");
}

int qe_moe_debug_set_epoch(qe_moe_ctx *c, uint32_t epoch, void *stream) {
    if (!c) return fail(QE_ERR_ARG, "debug_set_epoch: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    static uint32_t v;  // a pageable source is copied before hipMemcpyAsync returns
    v = epoch;
    HIP_TRY(hipMemcpyAsync(c->sync, &v, 4, hipMemcpyHostToDevice, (hipStream_t)stream));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return QE_OK;
}

int qe_moe_debug_fused_wait_extra(qe_moe_ctx *c, int extra) {
    if (!c || extra < 0) return fail(QE_ERR_ARG, "debug_fused_wait_extra: bad argument");
    c->S.wait_extra = extra;
    return QE_OK;
}

int qe_moe_debug_set_spin_cap(qe_moe_ctx *c, int cap) {
    if (!c || cap < 0) return fail(QE_ERR_ARG, "debug_set_spin_cap: bad argument");
    c->spin_cap = cap > 0 ? cap : QE_DECODE_SPIN_CAP;
    c->S.spin_cap = c->spin_cap;
    return QE_OK;
}

static const char *const k_prof_names[QP_N] = {
    "k_decode", "k_normq", "k_router_shgu", "unused", "k_topk",
    "k_disp_scatter", "k_expert_gu+k_expert_dn(+shared down)", "unused", "unused",
    "unused", "k_combine"};

int qe_moe_profile(qe_moe_ctx *c, int enable) {
    if (!c) return fail(QE_ERR_ARG, "profile: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    QeProf &p = c->prof;
    if (enable && !p.ev) {
        p.cap = 8192;
        p.ev = new hipEvent_t[2 * p.cap];
        p.kid = new int[p.cap];
        for (int i = 0; i < 2 * p.cap; ++i) HIP_TRY(hipEventCreate(&p.ev[i]));
    }
    p.on = enable != 0;
    p.used = 0;
    p.dropped = 0;
    return QE_OK;
}

int qe_moe_profile_read(qe_moe_ctx *c, double *ms, int *launches, int n) {
    if (!c || !ms || !launches || n < QP_N) return fail(QE_ERR_ARG, "profile_read: need arrays of %d", (int)QP_N);
    HIP_TRY(hipSetDevice(c->device));
    for (int k = 0; k < n; ++k) { ms[k] = 0.0; launches[k] = 0; }
    QeProf &p = c->prof;
    for (int i = 0; i < p.used; ++i) {
        HIP_TRY(hipEventSynchronize(p.ev[2 * i + 1]));
        float t = 0.f;
        HIP_TRY(hipEventElapsedTime(&t, p.ev[2 * i], p.ev[2 * i + 1]));
        ms[p.kid[i]] += t;
        launches[p.kid[i]] += 1;
    }
    const int dropped = p.dropped;
    p.used = 0;
    p.dropped = 0;
    if (dropped) return fail(QE_ERR_STATE, "profile_read: %d launches not recorded (event pool full)", dropped);
    return QE_OK;
}

const char *qe_moe_profile_name(int id) { return (id >= 0 && id < QP_N) ? k_prof_names[id] : ""; }

static size_t src_block_bytes(int type) {
    switch (type) {
    case QE_SRC_F32: return 128;
    case QE_SRC_F16: case QE_SRC_BF16: return 64;
    case QE_SRC_Q8_0: return 34;
    default: return 0;
    }
}

int qe_moe_nl4_quantize_rows(const void *src, int src_type, int64_t rows, int cols, void *dst, void *stream) {
    if (!src || !dst || rows < 0 || cols <= 0 || cols % 256 || ((uintptr_t)src | (uintptr_t)dst) % 16)
        return fail(QE_ERR_ARG, "nl4_quantize_rows: bad argument (rows=%lld cols=%d)", (long long)rows, cols);
    if (!src_block_bytes(src_type)) return fail(QE_ERR_ARG, "nl4_quantize_rows: unsupported source type %d", src_type);
    const int64_t nblk = rows * (cols / 32);
    if (nblk >= ((int64_t)1 << 31)) return fail(QE_ERR_ARG, "nl4_quantize_rows: %lld blocks (max 2^31 - 1)", (long long)nblk);
    QeNl4Args a;
    a.src = (const uint8_t *)src;
    a.dst = (uint8_t *)dst;
    a.nblk = (uint32_t)nblk;
    a.nb = (uint32_t)(cols / 32);
    a.rows_per_group = rows > 0 ? (uint32_t)rows : 1u;
    a.group_stride = 0;
    a.row_stride = QE_NL4_ROW_BYTES(cols);
    HIP_TRY(qe_launch_nl4_quant(a, src_type, (hipStream_t)stream));
    return QE_OK;
}

int qe_moe_convert_experts(qe_moe_ctx *c, int layer, const void *gate, const void *up, const void *down, int src_type,
                           void *stream) {
    if (!c || layer < 0 || layer >= c->n_layers || !gate || !up || !down ||
        ((uintptr_t)gate | (uintptr_t)up | (uintptr_t)down) % 16)
        return fail(QE_ERR_ARG, "convert_experts: bad argument");
    if (!src_block_bytes(src_type)) return fail(QE_ERR_ARG, "convert_experts: unsupported source type %d", src_type);
    HIP_TRY(hipSetDevice(c->device));
    uint8_t *base = c->arena + (size_t)layer * QE_LAYER_EXPERT_BYTES;
    QeNl4Args a;
    a.group_stride = QE_EXPERT_BYTES;
    // gate and up: 256 x 512 rows of 64 blocks
    a.nb = QE_D / 32;
    a.rows_per_group = QE_FF_EXP;
    a.nblk = QE_N_EXPERT * QE_FF_EXP * a.nb;
    a.row_stride = QE_GU_ROW_BYTES;
    a.src = (const uint8_t *)gate;
    a.dst = base;
    HIP_TRY(qe_launch_nl4_quant(a, src_type, (hipStream_t)stream));
    a.src = (const uint8_t *)up;
    a.dst = base + (size_t)QE_FF_EXP * QE_GU_ROW_BYTES;
    HIP_TRY(qe_launch_nl4_quant(a, src_type, (hipStream_t)stream));
    // down: 256 x 2048 rows of 16 blocks
    a.nb = QE_FF_EXP / 32;
    a.rows_per_group = QE_D;
    a.nblk = QE_N_EXPERT * QE_D * a.nb;
    a.row_stride = QE_DN_ROW_BYTES;
    a.src = (const uint8_t *)down;
    a.dst = base + QE_EXPERT_DOWN_OFF;
    HIP_TRY(qe_launch_nl4_quant(a, src_type, (hipStream_t)stream));
    mark_experts(c, layer, 0, QE_N_EXPERT);
    return QE_OK;
}

int qe_moe_arena_ptr(qe_moe_ctx *c, int layer, void **dev) {
    if (!c || !dev || layer < 0 || layer >= c->n_layers) return fail(QE_ERR_ARG, "arena_ptr: bad argument");
    *dev = c->arena + (size_t)layer * QE_LAYER_EXPERT_BYTES;
    mark_experts(c, layer, 0, QE_N_EXPERT); // the caller fills the arena in place
    return QE_OK;
}

int qe_moe_synth_layer(qe_moe_ctx *c, int layer, uint64_t seed, const float *bias, void *stream) {
    if (!c || layer < 0 || layer >= c->n_layers) return fail(QE_ERR_ARG, "synth_layer: bad argument");
    HIP_TRY(hipSetDevice(c->device));
    const QeLayerPtrs L = layer_ptrs(c, layer);
    HIP_TRY(qe_launch_synth_layer((uint8_t *)L.arena, (float *)L.router, (uint8_t *)L.sh_gu, (uint8_t *)L.sh_dn,
                                  (float *)L.post_norm, seed, layer, (hipStream_t)stream));
    if (bias) {
        HIP_TRY(hipMemcpyAsync(c->bias + (size_t)layer * QE_N_EXPERT, bias, QE_N_EXPERT * 4, hipMemcpyHostToDevice,
                               (hipStream_t)stream));
        c->has_bias[layer] = 1;
    } else {
        c->has_bias[layer] = 0;
    }
    HIP_TRY(hipMemcpyAsync(c->bias_on + layer, &c->has_bias[layer], 1, hipMemcpyHostToDevice, (hipStream_t)stream));
    HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    c->have[layer] = HAVE_ALL_DENSE;
    mark_experts(c, layer, 0, QE_N_EXPERT);
    return QE_OK;
}

int qe_moe_synth_zipf_bias(uint64_t seed, int layer, double s, float *out) {
    if (!out || !(s >= 0.0)) return fail(QE_ERR_ARG, "synth_zipf_bias: bad argument");
    qe_synth_zipf_bias(seed, layer, s, out);
    return QE_OK;
}

int qe_moe_synth_x(uint64_t seed, int inst, float *dev_out, int64_t n, void *stream) {
    if (!dev_out || n < 0) return fail(QE_ERR_ARG, "synth_x: bad argument");
    if (n == 0) return QE_OK;
    HIP_TRY(qe_launch_synth_x(dev_out, seed, inst, n, (hipStream_t)stream));
    return QE_OK;
}

}  // extern "C"
