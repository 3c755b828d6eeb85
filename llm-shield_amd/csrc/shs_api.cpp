// libshieldstral_hip host runtime: the C ABI of include/shieldstral_hip.h.
//
// Owns device memory, one HIP stream per handle, the KV cache and the forward-pass
// orchestration of MinistralModel.ForwardAsync (MinistralModel.cs:183-271), issuing
// the gfx950 kernels of shs_kernels.hip. No CPU fallback exists: without a gfx950
// device every entry point that needs one fails with SHS_E_DEVICE.
#include "shieldstral_hip.h"
#include "shs_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>
#include <ctime>

using namespace shs;

// ----------------------------------------------------------------- errors

static thread_local std::string g_error;

static shs_status fail(shs_status code, const char* fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

static shs_status hip_fail(hipError_t e, const char* what)
{
    return fail(SHS_E_DEVICE, "%s failed: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

#define HIP_TRY(expr)                                            \
    do {                                                         \
        hipError_t e_ = (expr);                                  \
        if (e_ != hipSuccess) return hip_fail(e_, #expr);        \
    } while (0)

extern "C" const char* shs_last_error(void) { return g_error.c_str(); }

// ------------------------------------------------------------- device bufs

namespace {

struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
    ~Buf() { release(); }
    void release()
    {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    hipError_t ensure(size_t n)
    {
        if (n <= bytes) return hipSuccess;
        release();
        hipError_t e = hipMalloc(&p, n);
        if (e == hipSuccess) bytes = n;
        else p = nullptr;
        return e;
    }
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Pinned host memory (hipHostMalloc), for the staging of small uploads.
struct HostBuf {
    void* p = nullptr;
    size_t bytes = 0;
    ~HostBuf() { release(); }
    void release()
    {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
    hipError_t ensure(size_t n)
    {
        if (n <= bytes) return hipSuccess;
        release();
        hipError_t e = hipHostMalloc(&p, n, hipHostMallocDefault);
        if (e == hipSuccess) bytes = n;
        else p = nullptr;
        return e;
    }
};

struct ActBuf {
    Buf all;  // act_q8_view's layout
    hipError_t ensure(int T, int K, ActQ8* view)
    {
        hipError_t e = all.ensure(act_q8_bytes(T, K));
        if (e != hipSuccess) return e;
        *view = act_q8_view(all.p, T, K);
        return hipSuccess;
    }
};

void free_matrix(DevMatrix& m)
{
    if (m.qs) (void)hipFree(m.qs);
    if (m.qh) (void)hipFree(m.qh);
    if (m.d) (void)hipFree(m.d);
    if (m.m) (void)hipFree(m.m);
    m = DevMatrix();
}

// Allocates a repacked matrix and clears it on stream s, the stream its rows are then
// uploaded on: a clear on another stream (hipMemset runs on the null stream, which a
// non-blocking stream does not wait for) could land after the repack and erase it.
hipError_t alloc_matrix(DevMatrix& m, int type, int rows, int cols, hipStream_t s)
{
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    m.blocks = cols / 32;
    m.tiles = (rows + 31) / 32;
    size_t recs = (size_t)m.tiles * m.blocks;
    hipError_t e;
    if ((e = hipMalloc((void**)&m.qs, recs * 32 * qs_bytes(type))) != hipSuccess) return e;
    if ((e = hipMemsetAsync(m.qs, 0, recs * 32 * qs_bytes(type), s)) != hipSuccess) return e;
    if ((e = hipMalloc((void**)&m.d, recs * 32 * sizeof(float))) != hipSuccess) return e;
    if ((e = hipMemsetAsync(m.d, 0, recs * 32 * sizeof(float), s)) != hipSuccess) return e;
    if (type_has_qh(type)) {
        if ((e = hipMalloc((void**)&m.qh, recs * 32 * sizeof(uint32_t))) != hipSuccess) return e;
        if ((e = hipMemsetAsync(m.qh, 0, recs * 32 * sizeof(uint32_t), s)) != hipSuccess) return e;
    }
    if (type_has_offset(type)) {
        if ((e = hipMalloc((void**)&m.m, recs * 32 * sizeof(float))) != hipSuccess) return e;
        if ((e = hipMemsetAsync(m.m, 0, recs * 32 * sizeof(float), s)) != hipSuccess) return e;
    }
    return hipSuccess;
}

int64_t row_bytes(int type, int64_t cols)
{
    int ts = type == SHS_Q4_0 ? 18 : type == SHS_Q4_1 ? 20 : type == SHS_Q5_0 ? 22 : type == SHS_Q5_1 ? 24
           : type == SHS_Q8_0 ? 34 : -1;
    return ts < 0 ? -1 : cols / 32 * ts;
}

const char* type_name(int t)
{
    switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    default: return "unsupported";
    }
}

// Where a tensor's native bytes come from: the caller's host buffer, or the synthetic
// generator (N(mean, std) quantized on the device) when host is null.
struct Source {
    const void* host = nullptr;
    uint64_t seed = 0, id = 0;
    float mean = 0.0f, std = 0.0f;
};

// Uploads (or generates) a native-layout tensor into rows [row0, row0+nrows) of a
// repacked matrix through a device staging buffer.
hipError_t upload_rows(DevMatrix& m, const Source& src, int row0, int nrows, Buf& staging, hipStream_t s)
{
    size_t bytes = (size_t)nrows * (size_t)row_bytes(m.type, m.cols);
    hipError_t e;
    if ((e = staging.ensure(bytes)) != hipSuccess) return e;
    if (src.host)
        e = hipMemcpyAsync(staging.p, src.host, bytes, hipMemcpyHostToDevice, s);
    else
        e = launch_synth_native(m.type, src.seed, src.id, nrows, m.cols, src.mean, src.std, staging.as<uint8_t>(), s);
    if (e != hipSuccess) return e;
    if ((e = launch_repack(m, staging.as<uint8_t>(), row0, nrows, s)) != hipSuccess) return e;
    return hipStreamSynchronize(s);
}

Source host_src(const void* p)
{
    Source s;
    s.host = p;
    return s;
}

bool device_is_gfx950(int device, std::string* arch)
{
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
    *arch = prop.gcnArchName;
    return arch->rfind("gfx950", 0) == 0;
}

shs_status select_device(int device)
{
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(SHS_E_DEVICE, "no HIP device is visible (%s); libshieldstral_hip runs only on a gfx950 (MI355X) GPU",
                    hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(SHS_E_INVALID_ARGUMENT, "device %d does not exist (%d visible)", device, count);
    std::string arch;
    if (!device_is_gfx950(device, &arch))
        return fail(SHS_E_DEVICE, "device %d is %s; these kernels are built for gfx950 (MI355X) only", device, arch.c_str());
    HIP_TRY(hipSetDevice(device));
    return SHS_OK;
}

// Kernel-class timing with events on the launching stream.
struct Profiler {
    bool on = false;
    struct Rec {
        hipEvent_t a, b;
        std::string cls, cls2;  // one event pair, counted under one or two classes
        double ops;
    };
    std::vector<Rec> pending;
    std::map<std::string, std::pair<int64_t, std::pair<double, double>>> totals;
    std::vector<hipEvent_t> pool;
    hipEvent_t get()
    {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    void begin(const char* cls, const char* cls2, double ops, hipStream_t s, Rec* r)
    {
        r->a = get();
        r->b = get();
        r->cls = cls;
        r->cls2 = cls2 ? cls2 : "";
        r->ops = ops;
        if (r->a) (void)hipEventRecord(r->a, s);
    }
    void end(Rec& r, hipStream_t s)
    {
        if (r.b) (void)hipEventRecord(r.b, s);
        pending.push_back(r);
    }
    void collect()
    {
        for (auto& r : pending) {
            float ms = 0.0f;
            if (r.a && r.b && hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
                for (const std::string* c : {&r.cls, &r.cls2}) {
                    if (c->empty()) continue;
                    auto& t = totals[*c];
                    t.first += 1;
                    t.second.first += ms;
                    t.second.second += r.ops;
                }
            }
            if (r.a) pool.push_back(r.a);
            if (r.b) pool.push_back(r.b);
        }
        pending.clear();
    }
    ~Profiler()
    {
        for (auto& r : pending) {
            if (r.a) (void)hipEventDestroy(r.a);
            if (r.b) (void)hipEventDestroy(r.b);
        }
        for (auto e : pool) (void)hipEventDestroy(e);
    }
};

// RAII scope that times one launch when profiling is on.
// Algorithmic HBM bytes of one RMSNorm + quantization launch over `rows` rows of n: the
// rows and the gains read, the int8 codes and per 32-block d, d·Σq and the 8-byte
// conversion column written.
static double rmsnorm_bytes(int rows, int n)
{
    return (double)rows * n * 4.0 + (double)n * 4.0 + (double)rows * n + (double)rows * (n / 32) * 16.0;
}

struct Timed {
    Profiler& p;
    hipStream_t s;
    Profiler::Rec rec{};
    bool active;
    Timed(Profiler& pr, const char* cls, double ops, hipStream_t st, const char* cls2 = nullptr)
        : p(pr), s(st), active(pr.on)
    {
        if (active) p.begin(cls, cls2, ops, s, &rec);
    }
    ~Timed()
    {
        if (active) p.end(rec, s);
    }
};

// A projection applied as one or more GEMMs writing adjacent column ranges of one
// output (q|k|v and gate|up are fused into one matrix when their types agree).
struct Proj {
    std::vector<DevMatrix> parts;
    std::vector<int> col0;
    int out_cols = 0;
};

// Where a named tensor lives on the device (for shs_tensor_download).
struct TensorLoc {
    const DevMatrix* mat = nullptr;  // matrices: rows [row0, row0 + rows) of mat
    int row0 = 0, rows = 0;
    const float* vec = nullptr;      // norm gains: n floats
    int n = 0;
};

struct Layer {
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    Proj qkv, o, gu, down;
};

}  // namespace

struct shs_matrix {
    DevMatrix w;
    int device = 0;
    hipStream_t stream = nullptr;
    ActBuf act;
    Buf x, y, ids, sums;
};

struct shs_model {
    shs_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    DevMatrix embd;
    DevMatrix head;  // output.weight when present; otherwise the tied embedding
    bool tied = true;
    float* out_norm = nullptr;
    std::vector<Layer> layers;
    // KV cache: per layer [kv_head][cap][head_dim] fp32, keys then values.
    float* kc = nullptr;
    float* vc = nullptr;
    int cap = 0, len = 0;
    // RoPE tables (host-computed cos/sin of position·freq, Rope.cs:117-122).
    std::vector<float> freqs;
    float mscale = 1.0f;
    int rope_cap = 0;
    Buf cos_tab, sin_tab, qscale_tab;
    // Work buffers, grown on demand.
    Buf h, qkv, ctx, gu, tmp, normed, ffn_act, tokens, pos, items, ids, logits, last_rows, lastidx, bkc, bvc, scores;
    // Attention work placed by place_items: the score kernel's key-tile chunks and the
    // scratch split into score tiles and per-tile row maxima.
    Buf chunks, counters;  // counters: the attention kernels' three work counters
    int n_chunks = 0;
    int n_cu = 0;          // compute units of the device (persistent kernel sizing)
    int fused_kt = 0;      // score tiles a fused-kernel block can hold in its LDS (a longer item spills the rest)
    int max_kt = 0;        // key tiles of the longest placed item
    int max_kt_fused = 0;  // key tiles of the longest item the fused kernel takes
    int n_long = 0;        // placed items past ATT_FUSED_MAX_KT key tiles: the first n_long of the list
    int max_lds = 0;       // LDS bytes a block may use (opt-in)
    int max_qc = 0;        // queries of the widest placed item
    int max_keys = 0;      // keys of the longest placed item
    int64_t score_floats = 0, pm_floats = 0;
    int64_t attn_pairs = 0, attn_pairs_long = 0;
    ActBuf act;
    ActBuf act_ffn;  // the fused gate|up GEMM's output codes (its input codes live in act)
    HostBuf stage;   // pinned staging of a call's small uploads (upload())
    size_t stage_used = 0;
    shs_capture_fn cap_fn = nullptr;
    void* cap_user = nullptr;
    Profiler prof;
    std::map<std::string, TensorLoc> where;
    // One completion event per layer, recorded when a pass can be cancelled (created on
    // first use): the host keeps at most CANCEL_LOOKAHEAD layers queued ahead of the GPU
    // and polls the flag while it waits for the oldest of them.
    std::vector<hipEvent_t> layer_done;
};

// ------------------------------------------------------------------ RoPE

static void rope_freqs(const shs_config& c, std::vector<float>& f, float& mscale)
{
    // Rope ctor (Rope.cs:33-66) and ComputeMagnitudeScale (Rope.cs:78-88).
    int dim = c.rope_dim, half = dim / 2;
    f.assign(half, 0.0f);
    float freq_scale = 1.0f / c.rope_scale;
    if (!c.yarn_active) {
        for (int i = 0; i < half; i++) f[i] = freq_scale / powf(c.rope_theta, 2.0f * (float)i / (float)dim);
        mscale = c.rope_attn_factor;
        return;
    }
    float low, high;
    if (c.yarn_beta_fast == 0.0f && c.yarn_beta_slow == 0.0f) {
        low = 3.40282347e38f;
        high = (float)dim / 2.0f - 1.0f;
    } else {
        const float PI = 3.14159265358979323846f;
        float cf = (float)dim * logf((float)c.rope_orig_ctx / (c.yarn_beta_fast * 2.0f * PI)) / (2.0f * logf(c.rope_theta));
        float cs = (float)dim * logf((float)c.rope_orig_ctx / (c.yarn_beta_slow * 2.0f * PI)) / (2.0f * logf(c.rope_theta));
        low = fmaxf(0.0f, floorf(cf));
        high = fminf((float)dim / 2.0f - 1.0f, ceilf(cs));
    }
    for (int i = 0; i < half; i++) {
        float extrapolated = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)dim);
        float interpolated = freq_scale * extrapolated;
        float y = ((float)i - low) / fmaxf(0.001f, high - low);
        float cl = y < 0.0f ? 0.0f : (y > 1.0f ? 1.0f : y);
        float mix = (1.0f - cl) * c.yarn_ext_factor;
        float a = interpolated * (1.0f - mix);
        float b = extrapolated * mix;
        f[i] = a + b;
    }
    auto ms = [](float scale, float m) { return scale <= 1.0f ? 1.0f : 0.1f * m * logf(scale) + 1.0f; };
    float factor = c.rope_scale;
    float m0 = c.yarn_mscale != 0.0f ? c.yarn_mscale : 1.0f;
    float ratio = c.yarn_mscale_all_dim != 0.0f ? ms(factor, m0) / ms(factor, c.yarn_mscale_all_dim) : ms(factor, 1.0f);
    mscale = ratio * c.rope_attn_factor;
}

static shs_status ensure_rope(shs_model* m, int need)
{
    if (need <= m->rope_cap) return SHS_OK;
    int cap = std::max(512, m->rope_cap);
    while (cap < need) cap *= 2;
    int half = m->cfg.rope_dim / 2;
    std::vector<float> c((size_t)cap * half), s((size_t)cap * half), qs(cap);
    for (int p = 0; p < cap; p++) {
        for (int i = 0; i < half; i++) {
            float theta = (float)p * m->freqs[i];
            c[(size_t)p * half + i] = cosf(theta) * m->mscale;
            s[(size_t)p * half + i] = sinf(theta) * m->mscale;
        }
        // ApplyPositionScale (MinistralModel.cs:476-482).
        float scale = 1.0f;
        if (m->cfg.rope_orig_ctx > 0 && m->cfg.attn_temperature != 0.0f) {
            float interval = floorf((float)p / (float)m->cfg.rope_orig_ctx);
            if (interval != 0.0f) scale = 1.0f + m->cfg.attn_temperature * logf(1.0f + interval);
        }
        qs[p] = scale;
    }
    HIP_TRY(m->cos_tab.ensure(c.size() * sizeof(float)));
    HIP_TRY(m->sin_tab.ensure(s.size() * sizeof(float)));
    HIP_TRY(m->qscale_tab.ensure(qs.size() * sizeof(float)));
    // Copied on the model's stream (which the kernels that read the tables run on) and
    // waited for before the host vectors go out of scope.
    HIP_TRY(hipMemcpyAsync(m->cos_tab.p, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice, m->stream));
    HIP_TRY(hipMemcpyAsync(m->sin_tab.p, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice, m->stream));
    HIP_TRY(hipMemcpyAsync(m->qscale_tab.p, qs.data(), qs.size() * sizeof(float), hipMemcpyHostToDevice, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    m->rope_cap = cap;
    return SHS_OK;
}

// ---------------------------------------------------------------- KV cache

static size_t kv_layer_floats(const shs_model* m, int cap)
{
    return (size_t)m->cfg.n_kv_head * cap * m->cfg.head_dim;
}

// KvCache.EnsureCapacity (KvCache.cs:48-70): doubles, keeping the first len positions.
static shs_status ensure_kv(shs_model* m, int need)
{
    if (need <= m->cap) return SHS_OK;
    int cap = std::max(1, m->cap);
    while (cap < need) cap *= 2;
    size_t per = kv_layer_floats(m, cap) * m->cfg.n_layer;
    float *kc = nullptr, *vc = nullptr;
    HIP_TRY(hipMalloc(&kc, per * sizeof(float)));
    hipError_t e = hipMalloc(&vc, per * sizeof(float));
    if (e != hipSuccess) {
        (void)hipFree(kc);
        return hip_fail(e, "hipMalloc(kv)");
    }
    if (m->len > 0 && m->kc) {
        size_t hd = m->cfg.head_dim;
        size_t rows = (size_t)m->cfg.n_layer * m->cfg.n_kv_head;
        HIP_TRY(hipMemcpy2DAsync(kc, cap * hd * 4, m->kc, m->cap * hd * 4, m->len * hd * 4, rows, hipMemcpyDeviceToDevice, m->stream));
        HIP_TRY(hipMemcpy2DAsync(vc, cap * hd * 4, m->vc, m->cap * hd * 4, m->len * hd * 4, rows, hipMemcpyDeviceToDevice, m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
    }
    if (m->kc) (void)hipFree(m->kc);
    if (m->vc) (void)hipFree(m->vc);
    m->kc = kc;
    m->vc = vc;
    m->cap = cap;
    return SHS_OK;
}

// ------------------------------------------------------------------ open

namespace {

// One tensor to load: its GGUF name, type, shape [ne0 = in, ne1 = out] and byte source.
struct Spec {
    std::string name;
    int type = 0;
    int64_t ne0 = 0, ne1 = 0;
    Source src;
};

struct SpecMap {
    std::map<std::string, Spec> byname;
    const Spec* get(const std::string& n) const
    {
        auto it = byname.find(n);
        return it == byname.end() ? nullptr : &it->second;
    }
};

shs_status need_tensor(const SpecMap& tm, const std::string& name, const Spec** out)
{
    *out = tm.get(name);
    if (!*out) return fail(SHS_E_KEY_NOT_FOUND, "tensor '%s' is missing; this does not look like a Shieldstral GGUF", name.c_str());
    return SHS_OK;
}

shs_status check_matrix(const Spec* t, int64_t in, int64_t out)
{
    if (!type_supported(t->type))
        return fail(SHS_E_NOT_SUPPORTED,
                    "tensor '%s' is %s; the integer GEMM takes Q4_0, Q4_1, Q5_0, Q5_1 and Q8_0 weights only",
                    t->name.c_str(), type_name(t->type));
    if (t->ne0 != in || t->ne1 != out)
        return fail(SHS_E_INVALID_DATA, "tensor '%s' is [%lld x %lld]; the model's hyperparameters need [%lld x %lld]",
                    t->name.c_str(), (long long)t->ne0, (long long)t->ne1, (long long)in, (long long)out);
    return SHS_OK;
}

shs_status load_proj(shs_model* m, Proj& p, const std::vector<const Spec*>& ts, Buf& staging)
{
    bool same = true;
    for (auto* t : ts) same = same && t->type == ts[0]->type;
    int total = 0;
    bool aligned = true;
    for (auto* t : ts) {
        aligned = aligned && total % 32 == 0;
        total += (int)t->ne1;
    }
    p.out_cols = total;
    p.parts.reserve(ts.size());
    if (same && aligned) {
        DevMatrix w;
        HIP_TRY(alloc_matrix(w, ts[0]->type, total, (int)ts[0]->ne0, m->stream));
        p.parts.push_back(w);
        p.col0.push_back(0);
        int row0 = 0;
        for (auto* t : ts) {
            HIP_TRY(upload_rows(p.parts[0], t->src, row0, (int)t->ne1, staging, m->stream));
            row0 += (int)t->ne1;
        }
        row0 = 0;
        for (auto* t : ts) {
            m->where[t->name] = TensorLoc{&p.parts[0], row0, (int)t->ne1, nullptr, 0};
            row0 += (int)t->ne1;
        }
    } else {
        int c0 = 0;
        for (auto* t : ts) {
            DevMatrix w;
            HIP_TRY(alloc_matrix(w, t->type, (int)t->ne1, (int)t->ne0, m->stream));
            p.parts.push_back(w);
            HIP_TRY(upload_rows(p.parts.back(), t->src, 0, (int)t->ne1, staging, m->stream));
            p.col0.push_back(c0);
            c0 += (int)t->ne1;
        }
        for (size_t i = 0; i < ts.size(); i++)
            m->where[ts[i]->name] = TensorLoc{&p.parts[i], 0, (int)ts[i]->ne1, nullptr, 0};
    }
    return SHS_OK;
}

shs_status upload_vector(shs_model* m, const Spec* t, int64_t n, float** out)
{
    if (t->ne0 != n || t->ne1 != 1)
        return fail(SHS_E_INVALID_DATA, "tensor '%s' has %lld elements; expected %lld", t->name.c_str(), (long long)(t->ne0 * t->ne1),
                    (long long)n);
    HIP_TRY(hipMalloc(out, n * sizeof(float)));
    if (!t->src.host) {
        HIP_TRY(launch_synth_f32(t->src.seed, t->src.id, n, t->src.mean, t->src.std, *out, m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
    } else {
        std::vector<float> v(n);
        if (t->type == SHS_F32) {
            memcpy(v.data(), t->src.host, n * sizeof(float));
        } else if (t->type == SHS_F16) {
            const uint16_t* h = static_cast<const uint16_t*>(t->src.host);
            for (int64_t i = 0; i < n; i++) {
                _Float16 x;
                memcpy(&x, &h[i], 2);
                v[i] = (float)x;
            }
        } else {
            return fail(SHS_E_NOT_SUPPORTED, "norm tensor '%s' is %s; F32 or F16 expected", t->name.c_str(), type_name(t->type));
        }
        HIP_TRY(hipMemcpyAsync(*out, v.data(), n * sizeof(float), hipMemcpyHostToDevice, m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
    }
    m->where[t->name] = TensorLoc{nullptr, 0, 0, *out, (int)n};
    return SHS_OK;
}

void destroy_model(shs_model* m)
{
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    free_matrix(m->embd);
    if (!m->tied) free_matrix(m->head);
    if (m->out_norm) (void)hipFree(m->out_norm);
    for (auto& L : m->layers) {
        if (L.attn_norm) (void)hipFree(L.attn_norm);
        if (L.ffn_norm) (void)hipFree(L.ffn_norm);
        for (Proj* p : {&L.qkv, &L.o, &L.gu, &L.down})
            for (auto& w : p->parts) free_matrix(w);
    }
    if (m->kc) (void)hipFree(m->kc);
    if (m->vc) (void)hipFree(m->vc);
    for (hipEvent_t e : m->layer_done) (void)hipEventDestroy(e);
    hipStream_t s = m->stream;
    delete m;
    if (s) (void)hipStreamDestroy(s);
}

shs_status check_config(const shs_config& c)
{
    if (c.n_layer <= 0 || c.hidden <= 0 || c.n_head <= 0 || c.n_kv_head <= 0 || c.head_dim <= 0 || c.ffn <= 0 || c.vocab <= 0)
        return fail(SHS_E_INVALID_DATA, "model hyperparameters must be positive");
    if (c.n_head % c.n_kv_head != 0)
        return fail(SHS_E_INVALID_DATA, "%d attention heads do not divide into %d KV heads.", c.n_head, c.n_kv_head);
    if (c.head_dim != 128 || c.n_head / c.n_kv_head > 4)
        return fail(SHS_E_NOT_SUPPORTED, "the attention kernel needs head_dim 128 and at most 4 query heads per KV head "
                                         "(got %d and %d)", c.head_dim, c.n_head / c.n_kv_head);
    if (c.hidden % 32 || c.ffn % 32 || c.rope_dim > c.head_dim || c.rope_dim <= 0 || c.rope_dim % 2)
        return fail(SHS_E_INVALID_DATA, "hidden and ffn must be multiples of 32 and rope_dim an even number ≤ head_dim");
    return SHS_OK;
}

// MinistralModel's constructor (MinistralModel.cs:59-108) over a set of tensor specs.
shs_status build_model(const shs_config& c, const SpecMap& tm, int device, int initial_capacity, shs_model** out)
{
    shs_status st = check_config(c);
    if (st != SHS_OK) return st;
    if ((st = select_device(device)) != SHS_OK) return st;
    shs_model* m = new shs_model();
    m->cfg = c;
    m->cfg.architecture[sizeof m->cfg.architecture - 1] = 0;
    if (!m->cfg.architecture[0]) snprintf(m->cfg.architecture, sizeof m->cfg.architecture, "mistral3");
    m->device = device;
    auto bail = [&](shs_status s) {
        std::string keep = g_error;
        destroy_model(m);
        g_error = keep;
        return s;
    };
    hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return bail(hip_fail(e, "hipStreamCreate"));
    if ((e = hipDeviceGetAttribute(&m->n_cu, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess)
        return bail(hip_fail(e, "hipDeviceGetAttribute"));
    {
        // the LDS a block may use once it asks for it (opt-in), else the default limit
        int optin = 0, base = 0;
        if ((e = hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, device)) != hipSuccess) optin = 0;
        if ((e = hipDeviceGetAttribute(&base, hipDeviceAttributeMaxSharedMemoryPerBlock, device)) != hipSuccess)
            return bail(hip_fail(e, "hipDeviceGetAttribute"));
        m->max_lds = std::max(optin, base);
        m->fused_kt = attn_fused_kt_limit(m->max_lds);
    }
    if ((e = m->counters.ensure(64)) != hipSuccess) return bail(hip_fail(e, "hipMalloc(counters)"));
    m->layers.reserve(c.n_layer);

    const int qdim = c.n_head * c.head_dim, kvdim = c.n_kv_head * c.head_dim;
    Buf staging;
    const Spec* t;
    if ((st = need_tensor(tm, "token_embd.weight", &t)) != SHS_OK) return bail(st);
    if ((st = check_matrix(t, c.hidden, c.vocab)) != SHS_OK) return bail(st);
    if ((e = alloc_matrix(m->embd, t->type, c.vocab, c.hidden, m->stream)) != hipSuccess) return bail(hip_fail(e, "hipMalloc(token_embd)"));
    if ((e = upload_rows(m->embd, t->src, 0, c.vocab, staging, m->stream)) != hipSuccess) return bail(hip_fail(e, "upload token_embd"));
    m->where[t->name] = TensorLoc{&m->embd, 0, c.vocab, nullptr, 0};
    // Shieldstral ties the LM head to token_embd; output.weight is used when present
    // (MinistralModel.cs:76-78, 250).
    const Spec* head = tm.get("output.weight");
    if (head) {
        if ((st = check_matrix(head, c.hidden, c.vocab)) != SHS_OK) return bail(st);
        if ((e = alloc_matrix(m->head, head->type, c.vocab, c.hidden, m->stream)) != hipSuccess) return bail(hip_fail(e, "hipMalloc(output)"));
        if ((e = upload_rows(m->head, head->src, 0, c.vocab, staging, m->stream)) != hipSuccess) return bail(hip_fail(e, "upload output"));
        m->tied = false;
        m->where[head->name] = TensorLoc{&m->head, 0, c.vocab, nullptr, 0};
    } else {
        m->head = m->embd;
        m->tied = true;
    }
    if ((st = need_tensor(tm, "output_norm.weight", &t)) != SHS_OK) return bail(st);
    if ((st = upload_vector(m, t, c.hidden, &m->out_norm)) != SHS_OK) return bail(st);

    m->layers.resize(c.n_layer);
    for (int l = 0; l < c.n_layer; l++) {
        Layer& L = m->layers[l];
        std::string p = "blk." + std::to_string(l) + ".";
        const Spec *an, *fn, *q, *k, *v, *o, *g, *u, *d;
        if ((st = need_tensor(tm, p + "attn_norm.weight", &an)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "attn_q.weight", &q)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "attn_k.weight", &k)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "attn_v.weight", &v)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "attn_output.weight", &o)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "ffn_norm.weight", &fn)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "ffn_gate.weight", &g)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "ffn_up.weight", &u)) != SHS_OK) return bail(st);
        if ((st = need_tensor(tm, p + "ffn_down.weight", &d)) != SHS_OK) return bail(st);
        if ((st = check_matrix(q, c.hidden, qdim)) != SHS_OK) return bail(st);
        if ((st = check_matrix(k, c.hidden, kvdim)) != SHS_OK) return bail(st);
        if ((st = check_matrix(v, c.hidden, kvdim)) != SHS_OK) return bail(st);
        if ((st = check_matrix(o, qdim, c.hidden)) != SHS_OK) return bail(st);
        if ((st = check_matrix(g, c.hidden, c.ffn)) != SHS_OK) return bail(st);
        if ((st = check_matrix(u, c.hidden, c.ffn)) != SHS_OK) return bail(st);
        if ((st = check_matrix(d, c.ffn, c.hidden)) != SHS_OK) return bail(st);
        if ((st = upload_vector(m, an, c.hidden, &L.attn_norm)) != SHS_OK) return bail(st);
        if ((st = upload_vector(m, fn, c.hidden, &L.ffn_norm)) != SHS_OK) return bail(st);
        if ((st = load_proj(m, L.qkv, {q, k, v}, staging)) != SHS_OK) return bail(st);
        if ((st = load_proj(m, L.o, {o}, staging)) != SHS_OK) return bail(st);
        if ((st = load_proj(m, L.gu, {g, u}, staging)) != SHS_OK) return bail(st);
        if ((st = load_proj(m, L.down, {d}, staging)) != SHS_OK) return bail(st);
    }
    rope_freqs(c, m->freqs, m->mscale);
    if ((st = ensure_kv(m, std::max(1, initial_capacity))) != SHS_OK) return bail(st);
    if ((st = ensure_rope(m, std::max(512, initial_capacity))) != SHS_OK) return bail(st);
    *out = m;
    return SHS_OK;
}

}  // namespace

extern "C" shs_status shs_open_tensors(const shs_config* cfg, const shs_tensor* tensors, int32_t n_tensors,
                                       int32_t device, int32_t initial_capacity, shs_model** out)
{
    if (!cfg || !out || (!tensors && n_tensors > 0)) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    SpecMap tm;
    for (int i = 0; i < n_tensors; i++) {
        const shs_tensor& t = tensors[i];
        if (!t.name) return fail(SHS_E_INVALID_ARGUMENT, "tensor %d has no name", i);
        if (!t.data) return fail(SHS_E_INVALID_ARGUMENT, "tensor '%s' has no data", t.name);
        Spec s;
        s.name = t.name;
        s.type = t.type;
        s.ne0 = t.ne0;
        s.ne1 = t.ne1 <= 0 ? 1 : t.ne1;
        s.src = host_src(t.data);
        tm.byname[s.name] = s;
    }
    return build_model(*cfg, tm, device, initial_capacity, out);
}

extern "C" shs_status shs_open_synthetic(const shs_config* cfg, int32_t weight_type, int32_t embd_type, uint64_t seed,
                                         int32_t device, int32_t initial_capacity, shs_model** out)
{
    if (!cfg || !out) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const shs_config& c = *cfg;
    if (c.n_layer <= 0) return fail(SHS_E_INVALID_DATA, "model hyperparameters must be positive");
    const int64_t qdim = (int64_t)c.n_head * c.head_dim, kvdim = (int64_t)c.n_kv_head * c.head_dim;
    SpecMap tm;
    uint64_t id = 0;
    auto add = [&](const std::string& name, int type, int64_t ne0, int64_t ne1, float mean, float std) {
        Spec s;
        s.name = name;
        s.type = type;
        s.ne0 = ne0;
        s.ne1 = ne1;
        s.src.seed = seed;
        s.src.id = id++;
        s.src.mean = mean;
        s.src.std = std;
        tm.byname[name] = s;
    };
    add("token_embd.weight", embd_type, c.hidden, c.vocab, 0.0f, 0.02f);
    add("output_norm.weight", SHS_F32, c.hidden, 1, 1.0f, 0.1f);
    for (int l = 0; l < c.n_layer; l++) {
        std::string p = "blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", SHS_F32, c.hidden, 1, 1.0f, 0.1f);
        add(p + "attn_q.weight", weight_type, c.hidden, qdim, 0.0f, 0.02f);
        add(p + "attn_k.weight", weight_type, c.hidden, kvdim, 0.0f, 0.02f);
        add(p + "attn_v.weight", weight_type, c.hidden, kvdim, 0.0f, 0.02f);
        add(p + "attn_output.weight", weight_type, qdim, c.hidden, 0.0f, 0.02f);
        add(p + "ffn_norm.weight", SHS_F32, c.hidden, 1, 1.0f, 0.1f);
        add(p + "ffn_gate.weight", weight_type, c.hidden, c.ffn, 0.0f, 0.02f);
        add(p + "ffn_up.weight", weight_type, c.hidden, c.ffn, 0.0f, 0.02f);
        add(p + "ffn_down.weight", weight_type, c.ffn, c.hidden, 0.0f, 0.02f);
    }
    return build_model(c, tm, device, initial_capacity, out);
}

extern "C" shs_status shs_tensor_download(shs_model* m, const char* name, void* dst, size_t bytes)
{
    if (!m || !name || !dst) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    auto it = m->where.find(name);
    if (it == m->where.end()) return fail(SHS_E_KEY_NOT_FOUND, "tensor '%s' is not part of this model", name);
    const TensorLoc& loc = it->second;
    HIP_TRY(hipSetDevice(m->device));
    if (loc.vec) {
        if (bytes != sizeof(float) * (size_t)loc.n)
            return fail(SHS_E_INVALID_ARGUMENT, "'%s' is %d fp32 values; buffer holds %zu bytes", name, loc.n, bytes);
        HIP_TRY(hipMemcpy(dst, loc.vec, bytes, hipMemcpyDeviceToHost));
        return SHS_OK;
    }
    size_t need = (size_t)loc.rows * (size_t)row_bytes(loc.mat->type, loc.mat->cols);
    if (bytes != need) return fail(SHS_E_INVALID_ARGUMENT, "'%s' is %zu bytes; buffer holds %zu", name, need, bytes);
    Buf tmp;
    HIP_TRY(tmp.ensure(need));
    HIP_TRY(launch_unpack_native(*loc.mat, loc.row0, loc.rows, tmp.as<uint8_t>(), m->stream));
    HIP_TRY(hipMemcpyAsync(dst, tmp.p, need, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" void shs_close(shs_model* m) { destroy_model(m); }

extern "C" shs_status shs_get_config(const shs_model* m, shs_config* out)
{
    if (!m || !out) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *out = m->cfg;
    return SHS_OK;
}

extern "C" shs_status shs_kv_reset(shs_model* m)
{
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null model");
    m->len = 0;
    return SHS_OK;
}

extern "C" shs_status shs_kv_length(const shs_model* m, int32_t* n)
{
    if (!m || !n) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *n = m->len;
    return SHS_OK;
}

extern "C" shs_status shs_kv_capacity(const shs_model* m, int32_t* n)
{
    if (!m || !n) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *n = m->cap;
    return SHS_OK;
}

extern "C" shs_status shs_kv_snapshot(shs_model* m, int32_t length, float* dst, size_t n_floats)
{
    if (!m || (!dst && length > 0)) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (length < 0 || length > m->len)
        return fail(SHS_E_OUT_OF_RANGE, "only %d positions are cached; cannot snapshot %d", m->len, length);
    size_t hd = m->cfg.head_dim, rows = (size_t)m->cfg.n_layer * m->cfg.n_kv_head;
    size_t per = rows * length * hd;
    if (n_floats != 2 * per)
        return fail(SHS_E_INVALID_ARGUMENT, "snapshot of %d positions holds %zu floats, buffer has %zu", length, 2 * per, n_floats);
    if (length == 0) return SHS_OK;
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(hipMemcpy2DAsync(dst, length * hd * 4, m->kc, m->cap * hd * 4, length * hd * 4, rows, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipMemcpy2DAsync(dst + per, length * hd * 4, m->vc, m->cap * hd * 4, length * hd * 4, rows, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_kv_restore(shs_model* m, const float* src, size_t n_floats, int32_t length)
{
    if (!m || (!src && length > 0)) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (length < 0) return fail(SHS_E_OUT_OF_RANGE, "negative length");
    size_t hd = m->cfg.head_dim, rows = (size_t)m->cfg.n_layer * m->cfg.n_kv_head;
    size_t per = rows * length * hd;
    if (n_floats != 2 * per)
        return fail(SHS_E_INVALID_ARGUMENT, "Snapshot holds %zu floats; %d positions need %zu.", n_floats, length, 2 * per);
    HIP_TRY(hipSetDevice(m->device));
    shs_status st = ensure_kv(m, length);
    if (st != SHS_OK) return st;
    if (length > 0) {
        HIP_TRY(hipMemcpy2DAsync(m->kc, m->cap * hd * 4, src, length * hd * 4, length * hd * 4, rows, hipMemcpyHostToDevice, m->stream));
        HIP_TRY(hipMemcpy2DAsync(m->vc, m->cap * hd * 4, src + per, length * hd * 4, length * hd * 4, rows, hipMemcpyHostToDevice, m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
    }
    m->len = length;
    return SHS_OK;
}

extern "C" shs_status shs_set_capture(shs_model* m, shs_capture_fn fn, void* user)
{
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null model");
    m->cap_fn = fn;
    m->cap_user = user;
    return SHS_OK;
}

// ------------------------------------------------------------- forward

namespace {

struct Capture {
    shs_model* m;
    std::vector<float> host;
    shs_status observe(const char* name, const float* dev, int ld, int rows, int cols)
    {
        if (!m->cap_fn) return SHS_OK;
        host.resize((size_t)rows * cols);
        HIP_TRY(hipStreamSynchronize(m->stream));
        HIP_TRY(hipMemcpy2D(host.data(), cols * sizeof(float), dev, ld * sizeof(float), cols * sizeof(float), rows,
                            hipMemcpyDeviceToHost));
        m->cap_fn(name, host.data(), rows, cols, m->cap_user);
        return SHS_OK;
    }
};

double gemm_ops(int T, const DevMatrix& w) { return 2.0 * T * (double)w.rows * w.cols; }

// Each launch is timed under the projection's class and under its kernel instantiation,
// "k_gemm<type,TT,mode,BPS>" (the name rocprofv3 reports, so the two can be compared).
// The name rocprofv3 reports for the GEMM kernel launch_gemm* picks for this shape and mode.
void gemm_kname(char* buf, size_t n, const DevMatrix& w, const ActQ8& a, int mode)
{
    const int nt = gemm_narrow_tokens(w, a, mode);
    if (nt > 0)
        snprintf(buf, n, "k_gemm_narrow<%d,%d,%d>", w.type, nt, mode);
    else {
        const int tt = gemm_token_tiles(w, a, mode);
        snprintf(buf, n, "k_gemm<%d,%d,%d,%d>", w.type, tt, mode, gemm_stage_blocks(w, tt));
    }
}

shs_status run_proj(shs_model* m, const Proj& p, const ActQ8& a, float* y, int ldy, int mode, const char* cls)
{
    for (size_t i = 0; i < p.parts.size(); i++) {
        const DevMatrix& w = p.parts[i];
        char kname[48] = "k_gemm";
        if (m->prof.on) gemm_kname(kname, sizeof kname, w, a, mode);
        Timed tm(m->prof, cls, gemm_ops(a.T, w), m->stream, kname);
        HIP_TRY(launch_gemm(w, a, y + p.col0[i], ldy, mode, m->stream));
    }
    return SHS_OK;
}

// Buffers for a pass over T tokens.
shs_status ensure_work(shs_model* m, int T)
{
    const shs_config& c = m->cfg;
    size_t qdim = (size_t)c.n_head * c.head_dim, kvdim = (size_t)c.n_kv_head * c.head_dim;
    HIP_TRY(m->h.ensure(sizeof(float) * T * c.hidden));
    HIP_TRY(m->qkv.ensure(sizeof(float) * T * (qdim + 2 * kvdim)));
    HIP_TRY(m->ctx.ensure(sizeof(float) * T * qdim));
    HIP_TRY(m->gu.ensure(sizeof(float) * T * 2 * (size_t)c.ffn));
    HIP_TRY(m->tmp.ensure(sizeof(float) * T * std::max<size_t>(c.hidden, c.ffn)));
    HIP_TRY(m->normed.ensure(sizeof(float) * T * (size_t)c.hidden));
    HIP_TRY(m->tokens.ensure(sizeof(int32_t) * T));
    HIP_TRY(m->pos.ensure(sizeof(int32_t) * T));
    return SHS_OK;
}

// Layers a cancellable pass queues ahead of the one the GPU is running: enough to keep
// the GPU fed between the host's polls, few enough that a cancel is seen within about
// two layers of execution (ModerationCancellationTests.cs:50-74).
constexpr int CANCEL_LOOKAHEAD = 2;

// Before layer l of a cancellable pass is queued: waits until layer l − CANCEL_LOOKAHEAD
// has run on the GPU, polling the flag meanwhile. Returns SHS_E_CANCELLED (after the
// queued layers drain) once the flag is set.
shs_status cancel_point(shs_model* m, int l, int l_begin, const volatile int32_t* cancel)
{
    auto cancelled = [&] {
        (void)hipStreamSynchronize(m->stream);
        return fail(SHS_E_CANCELLED, "The operation was canceled.");
    };
    if (*cancel) return cancelled();
    if (m->layer_done.empty()) {
        m->layer_done.assign(m->cfg.n_layer, nullptr);
        for (auto& e : m->layer_done) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const int wait_for = l - CANCEL_LOOKAHEAD;
    if (wait_for < l_begin) return SHS_OK;
    for (;;) {
        const hipError_t q = hipEventQuery(m->layer_done[wait_for]);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) return hip_fail(q, "hipEventQuery");
        if (*cancel) return cancelled();
        struct timespec ts = {0, 20000};  // 20 µs between polls
        nanosleep(&ts, nullptr);
    }
    return *cancel ? cancelled() : SHS_OK;
}

// The decoder layers over the T tokens in m->h. Keys and values for token t go to cache
// slot slot0 + t of (kc, vc) whose per-head stride is cap positions; attention runs over
// the given work items. With a cancel flag, at most CANCEL_LOOKAHEAD layers are queued
// ahead of the GPU and the flag is polled while the host waits for them, so a cancel
// set during execution is observed between layers.
shs_status run_layers(shs_model* m, int T, float* kc_all, float* vc_all, int cap, int slot0, int l_begin, int l_end,
                      const AttnItem* items_dev, int n_items, const volatile int32_t* cancel, bool per_layer_kv)
{
    const shs_config& c = m->cfg;
    const int hidden = c.hidden, qdim = c.n_head * c.head_dim, kvdim = c.n_kv_head * c.head_dim;
    const int ldqkv = qdim + 2 * kvdim;
    float* h = m->h.as<float>();
    float* qkv = m->qkv.as<float>();
    float* ctx = m->ctx.as<float>();
    float* gu = m->gu.as<float>();
    float* tmp = m->tmp.as<float>();
    const bool cap_on = m->cap_fn != nullptr;
    float* normed = cap_on ? m->normed.as<float>() : nullptr;
    Capture cp{m, {}};
    char name[96];
    const float scale = 1.0f / sqrtf((float)c.head_dim);
    ActQ8 a;
    HIP_TRY(m->act.ensure(T, std::max(std::max(hidden, qdim), c.ffn), &a));

    for (int l = l_begin; l < l_end; l++) {
        if (cancel) {
            shs_status cs = cancel_point(m, l, l_begin, cancel);
            if (cs != SHS_OK) return cs;
        }
        const Layer& L = m->layers[l];
        float* kc = per_layer_kv ? kc_all + kv_layer_floats(m, cap) * l : kc_all;
        float* vc = per_layer_kv ? vc_all + kv_layer_floats(m, cap) * l : vc_all;

        ActQ8 ah = a;
        ah.K = hidden;
        ah.B = hidden / 32;
        // At decode width the fused q|k|v and gate|up kernels normalize and quantize the hidden
        // rows themselves (NormIn); otherwise k_rmsnorm_quant writes the codes first.
        NormIn attn_in, ffn_in;
        attn_in.x = ffn_in.x = h;
        attn_in.ldx = ffn_in.ldx = hidden;
        attn_in.eps = ffn_in.eps = c.rms_eps;
        attn_in.w = L.attn_norm;
        ffn_in.w = L.ffn_norm;
        const bool qkv_fused = !cap_on && L.qkv.parts.size() == 1 && c.head_dim % 32 == 0;
        const bool gu_fused = !cap_on && L.gu.parts.size() == 1;
        const bool qkv_norm = qkv_fused && gemm_narrow_tokens(L.qkv.parts[0], ah, GEMM_QKV, true) > 0;
        const bool gu_norm = gu_fused && gemm_narrow_tokens(L.gu.parts[0], ah, GEMM_SWIGLU, true) > 0;
        if (!qkv_norm) {
            Timed tm(m->prof, "rmsnorm_quant", rmsnorm_bytes(T, hidden), m->stream);
            HIP_TRY(launch_rmsnorm_quant(h, hidden, L.attn_norm, c.rms_eps, hidden, ah, normed, m->stream));
        }
        snprintf(name, sizeof name, "blk.%d.attn_norm", l);
        if (cap_on && cp.observe(name, normed, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;

        if (qkv_fused) {
            // one fused matrix: RoPE and the KV-cache store in the epilogue
            RopeArgs ra;
            ra.pos = m->pos.as<int32_t>();
            ra.ct = m->cos_tab.as<float>();
            ra.st = m->sin_tab.as<float>();
            ra.qscale = m->qscale_tab.as<float>();
            ra.half = c.rope_dim / 2;
            ra.n_head = c.n_head;
            ra.n_kv = c.n_kv_head;
            ra.hd = c.head_dim;
            ra.kc = kc;
            ra.vc = vc;
            ra.cap = cap;
            ra.slot0 = slot0;
            const DevMatrix& w = L.qkv.parts[0];
            char kname[48] = "k_gemm";
            if (m->prof.on) gemm_kname(kname, sizeof kname, w, ah, GEMM_QKV);
            Timed tm(m->prof, "gemm_qkv", gemm_ops(T, w), m->stream, kname);
            HIP_TRY(launch_gemm_qkv(w, ah, qkv, ldqkv, ra, m->stream, qkv_norm ? &attn_in : nullptr));
        } else {
            if (run_proj(m, L.qkv, ah, qkv, ldqkv, GEMM_STORE, "gemm_qkv") != SHS_OK) return SHS_E_DEVICE;
            Timed tm(m->prof, "rope_store", 0, m->stream);
            HIP_TRY(launch_rope_store(qkv, ldqkv, T, c.n_head, c.n_kv_head, c.head_dim, m->pos.as<int32_t>(),
                                      m->cos_tab.as<float>(), m->sin_tab.as<float>(), m->qscale_tab.as<float>(),
                                      c.rope_dim / 2, kc, vc, cap, slot0, m->stream));
        }
        if (cap_on) {
            snprintf(name, sizeof name, "blk.%d.q_rope", l);
            if (cp.observe(name, qkv, ldqkv, T, qdim) != SHS_OK) return SHS_E_DEVICE;
            snprintf(name, sizeof name, "blk.%d.k_rope", l);
            if (cp.observe(name, qkv + qdim, ldqkv, T, kvdim) != SHS_OK) return SHS_E_DEVICE;
            snprintf(name, sizeof name, "blk.%d.v", l);
            if (cp.observe(name, qkv + qdim + kvdim, ldqkv, T, kvdim) != SHS_OK) return SHS_E_DEVICE;
        }
        ActQ8 ac = a;
        ac.K = qdim;
        ac.B = qdim / 32;
        {
            float* scr = m->scores.as<float>();
            float* pm = scr + m->score_floats;
            int* ctr = m->counters.as<int>();
            // 2·head_dim flops per (query, key) pair and head, for the scores and again for the values
            const double attn_ops = 2.0 * c.head_dim * c.n_head * (double)m->attn_pairs;
            const double long_ops = 2.0 * c.head_dim * c.n_head * (double)m->attn_pairs_long;
            if (m->max_qc <= ATT_DEC_MAX_Q && c.n_head / c.n_kv_head <= 4 &&
                m->max_keys <= attn_decode_max_keys(m->max_qc, m->max_lds)) {
                // decode width: scores per (KV head, 64-key chunk), values per (head, 32-dim slice)
                Timed tk(m->prof, "attn_decode", attn_ops, m->stream, "attention");
                HIP_TRY(launch_attn_decode(qkv, ldqkv, kc, vc, cap, items_dev, n_items, c.n_head, c.n_kv_head,
                                           c.head_dim, scale, m->max_qc, m->max_keys, scr, ctx, qdim,
                                           cap_on ? nullptr : &ac, m->stream));
            } else {
                // Items past ATT_FUSED_MAX_KT key tiles (the first n_long of the list) take the
                // three kernels through the score scratch; the rest the fused kernel, whose block
                // holds an item's first score tiles in its LDS and the rest in the item's scratch
                // region, and which, without capture, writes the o projection's activation codes
                // itself. The two sets of items write disjoint rows and regions.
                const int n_long = m->n_long, n_fused = n_items - n_long;
                if (n_long > 0) {
                    {
                        Timed tk(m->prof, "k_attn_scores", long_ops, m->stream, "attention");
                        HIP_TRY(launch_attn_scores(qkv, ldqkv, kc, cap, items_dev, m->chunks.as<AttnChunk>(),
                                                   m->n_chunks, c.n_head, c.n_kv_head, c.head_dim, scale, scr, pm,
                                                   m->stream));
                    }
                    {
                        Timed tk(m->prof, "k_attn_softmax", 0, m->stream, "attention");
                        HIP_TRY(launch_attn_softmax(items_dev, n_long, c.n_head, c.n_kv_head, scr, pm, ctr, m->n_cu,
                                                    m->stream));
                    }
                    {
                        Timed tk(m->prof, "k_attn_pv", long_ops, m->stream, "attention");
                        HIP_TRY(launch_attn_pv(vc, cap, items_dev, n_long, c.n_head, c.n_kv_head, scr, ctx, qdim,
                                               cap_on ? nullptr : &ac, ctr, m->n_cu, m->stream));
                    }
                }
                if (n_fused > 0) {
                    Timed tk(m->prof, "k_attn_fused", 2 * (attn_ops - long_ops), m->stream, "attention");
                    // the LDS holds up to fused_kt tiles; past them the spilling instantiation runs
                    const int kt_cap = std::min(m->max_kt_fused, m->fused_kt);
                    HIP_TRY(launch_attn_fused(qkv, ldqkv, kc, vc, cap, items_dev + n_long, n_fused, c.n_head,
                                              c.n_kv_head, c.head_dim, scale, ctx, qdim, cap_on ? nullptr : &ac, kt_cap,
                                              m->max_kt_fused > kt_cap ? scr : nullptr, m->stream));
                }
            }
        }
        snprintf(name, sizeof name, "blk.%d.attn_weighted", l);
        if (cap_on && cp.observe(name, ctx, qdim, T, qdim) != SHS_OK) return SHS_E_DEVICE;

        if (cap_on) {
            Timed tm(m->prof, "quant_act", 0, m->stream);
            HIP_TRY(launch_quant_act(ctx, qdim, ac, 0, m->stream));
        }
        if (cap_on) {
            if (run_proj(m, L.o, ac, tmp, hidden, GEMM_STORE, "gemm_o") != SHS_OK) return SHS_E_DEVICE;
            snprintf(name, sizeof name, "blk.%d.attn_out", l);
            if (cp.observe(name, tmp, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;
            HIP_TRY(launch_add_inplace(h, tmp, (size_t)T * hidden, m->stream));
            snprintf(name, sizeof name, "blk.%d.post_attn", l);
            if (cp.observe(name, h, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;
        } else {
            if (run_proj(m, L.o, ac, h, hidden, GEMM_ADD, "gemm_o") != SHS_OK) return SHS_E_DEVICE;
        }

        if (!gu_norm) {
            Timed tm(m->prof, "rmsnorm_quant", rmsnorm_bytes(T, hidden), m->stream);
            HIP_TRY(launch_rmsnorm_quant(h, hidden, L.ffn_norm, c.rms_eps, hidden, ah, normed, m->stream));
        }
        snprintf(name, sizeof name, "blk.%d.ffn_norm", l);
        if (cap_on && cp.observe(name, normed, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;

        ActQ8 af = a;
        af.K = c.ffn;
        af.B = c.ffn / 32;
        if (gu_fused) {
            // one fused matrix: SwiGLU and the down projection's quantization in the epilogue
            HIP_TRY(m->act_ffn.ensure(T, c.ffn, &af));
            const DevMatrix& w = L.gu.parts[0];
            char kname[48] = "k_gemm";
            if (m->prof.on) gemm_kname(kname, sizeof kname, w, ah, GEMM_SWIGLU);
            Timed tm(m->prof, "gemm_gate_up", gemm_ops(T, w), m->stream, kname);
            HIP_TRY(launch_gemm_swiglu(w, ah, c.ffn / 32, af, m->stream, gu_norm ? &ffn_in : nullptr));
        } else {
            if (run_proj(m, L.gu, ah, gu, 2 * c.ffn, GEMM_STORE, "gemm_gate_up") != SHS_OK) return SHS_E_DEVICE;
            Timed tm(m->prof, "swiglu_quant", 0, m->stream);
            HIP_TRY(launch_swiglu_quant(gu, 2 * c.ffn, c.ffn, af, nullptr, m->stream));
        }
        if (cap_on) {
            if (run_proj(m, L.down, af, tmp, hidden, GEMM_STORE, "gemm_down") != SHS_OK) return SHS_E_DEVICE;
            snprintf(name, sizeof name, "blk.%d.ffn_out", l);
            if (cp.observe(name, tmp, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;
            HIP_TRY(launch_add_inplace(h, tmp, (size_t)T * hidden, m->stream));
            snprintf(name, sizeof name, "blk.%d.output", l);
            if (cp.observe(name, h, hidden, T, hidden) != SHS_OK) return SHS_E_DEVICE;
        } else {
            if (run_proj(m, L.down, af, h, hidden, GEMM_ADD, "gemm_down") != SHS_OK) return SHS_E_DEVICE;
        }
        if (cancel) HIP_TRY(hipEventRecord(m->layer_done[l], m->stream));
    }
    return SHS_OK;
}

// Final RMSNorm of the rows `rows` of h, then the head: selected rows or the full vocab.
shs_status run_head(shs_model* m, const std::vector<int32_t>& rows, int head_mode, const int32_t* ids_dev, int n_ids,
                    float* logits_dev)
{
    const shs_config& c = m->cfg;
    const int n = (int)rows.size();
    HIP_TRY(m->normed.ensure(sizeof(float) * (size_t)std::max(n, 1) * c.hidden));
    // one row (a prompt's last token) is read in place; several are gathered first
    const float* x_in = m->h.as<float>() + (n == 1 ? (size_t)rows[0] * c.hidden : 0);
    if (n != 1) {
        HIP_TRY(m->lastidx.ensure(sizeof(int32_t) * n));
        HIP_TRY(m->last_rows.ensure(sizeof(float) * (size_t)n * c.hidden));
        HIP_TRY(hipMemcpyAsync(m->lastidx.p, rows.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice, m->stream));
        HIP_TRY(launch_gather_rows(m->h.as<float>(), c.hidden, m->lastidx.as<int32_t>(), n, c.hidden,
                                   m->last_rows.as<float>(), c.hidden, m->stream));
        x_in = m->last_rows.as<float>();
    }
    ActQ8 a;
    HIP_TRY(m->act.ensure(n, c.hidden, &a));
    float* normed = m->cap_fn ? m->normed.as<float>() : nullptr;
    {
        Timed tm(m->prof, "rmsnorm_quant", rmsnorm_bytes(n, c.hidden), m->stream);
        HIP_TRY(launch_rmsnorm_quant(x_in, c.hidden, m->out_norm, c.rms_eps, c.hidden, a, normed, m->stream));
    }
    Capture cp{m, {}};
    if (m->cap_fn && cp.observe("final_norm", normed, c.hidden, n, c.hidden) != SHS_OK) return SHS_E_DEVICE;
    if (head_mode == 1) {
        Timed tm(m->prof, "gemv", 2.0 * n * n_ids * c.hidden, m->stream);
        HIP_TRY(launch_gemv_rows(m->head, a, ids_dev, n_ids, logits_dev, m->stream));
    } else {
        Timed tm(m->prof, "gemm_head", gemm_ops(n, m->head), m->stream);
        HIP_TRY(launch_gemm(m->head, a, logits_dev, c.vocab, GEMM_STORE, m->stream));
    }
    return SHS_OK;
}

shs_status check_ids(const int32_t* ids, int n, int limit, const char* what)
{
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= limit)
            return fail(SHS_E_OUT_OF_RANGE, "%s %d is outside the %d-entry table.", what, ids[i], limit);
    return SHS_OK;
}

std::vector<AttnItem> causal_items(int q_begin, int n, int key_start, int pos0)
{
    std::vector<AttnItem> v;
    for (int k = 0; k * 32 < n; k++) v.push_back({q_begin + 32 * k, std::min(32, n - 32 * k), key_start, pos0 + 32 * k, 0});
    return v;
}

// A call's small uploads (token ids, positions, attention work) go through the pinned staging
// buffer, so their copies are asynchronous and the call queues its kernels without waiting for
// them. begin_uploads runs before a call's first upload and waits for the stream (idle then:
// every call synchronizes before it returns, an early error return included the next call's
// wait), so the buffer can be reused. An upload that does not fit is copied directly and
// waited for.
hipError_t begin_uploads(shs_model* m)
{
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) return e;
    m->stage_used = 0;
    return m->stage.ensure(256u << 10);
}

hipError_t upload(shs_model* m, void* dst, const void* src, size_t bytes)
{
    if (bytes == 0) return hipSuccess;
    if (m->stage.p && m->stage_used + bytes <= m->stage.bytes) {
        char* st = static_cast<char*>(m->stage.p) + m->stage_used;
        memcpy(st, src, bytes);
        m->stage_used += (bytes + 255) & ~(size_t)255;
        return hipMemcpyAsync(dst, st, bytes, hipMemcpyHostToDevice, m->stream);
    }
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, m->stream);
    return e != hipSuccess ? e : hipStreamSynchronize(m->stream);
}

// Orders the items for the attention kernels: those past the fused kernel's key tiles first,
// then those it takes, each group by ascending length (the kernels start from the end of
// their group, longest first). Gives every item its own region of the score scratch (4 waves
// per KV head, one 32×32 tile of 1024 floats per key tile), splits the long items' key tiles
// into the score kernel's chunks and sizes the scratch: score tiles, then 32 row maxima per
// tile.
// The chunk length c (2..8 key tiles) minimizes rounds × (c + 1): the score kernel's blocks
// fill its resident slots round by round, and a block costs about one tile more than its
// tiles for its own start (the q and first K loads). Ties go to the shorter chunk.
shs_status place_items(shs_model* m, std::vector<AttnItem>& items)
{
    auto tiles = [](const AttnItem& it) { return (it.pos0 + it.q_count + 31) / 32; };
    std::stable_sort(items.begin(), items.end(),
                     [&](const AttnItem& a, const AttnItem& b) { return tiles(a) < tiles(b); });
    // items past ATT_FUSED_MAX_KT key tiles take the three-kernel path; the fused kernel holds
    // up to fused_kt tiles of the rest in its LDS and their later tiles in their regions
    const int fused_max = m->fused_kt > 0 ? ATT_FUSED_MAX_KT : 0;
    std::stable_partition(items.begin(), items.end(), [&](const AttnItem& it) { return tiles(it) > fused_max; });
    int n_long = 0;
    while (n_long < (int)items.size() && tiles(items[n_long]) > fused_max) n_long++;
    int kChunk = 4;
    {
        const int64_t slots = std::max(1, attn_score_slots(m->n_cu));
        int64_t best = -1;
        for (int c = 2; c <= 8; c++) {
            int64_t blocks = 0;
            for (int i = 0; i < n_long; i++) blocks += (tiles(items[i]) + c - 1) / c;
            blocks *= m->cfg.n_kv_head;
            const int64_t cost = (blocks + slots - 1) / slots * (c + 1);
            if (best < 0 || cost < best) {
                best = cost;
                kChunk = c;
            }
        }
    }
    // every item gets a region: the decode-width kernels keep their scores there too
    int64_t off = 0;
    for (auto& it : items) {
        it.s_off = off;
        off += (int64_t)tiles(it) * 1024 * (int64_t)m->cfg.n_kv_head * 4;
    }
    std::vector<AttnChunk> chunks;
    for (int i = n_long - 1; i >= 0; i--) {
        const int n_kt = tiles(items[i]);
        for (int k = 0; k < n_kt; k += kChunk) chunks.push_back({i, k, std::min(kChunk, n_kt - k), 0});
    }
    m->score_floats = off;
    m->pm_floats = off / 32;
    m->n_long = n_long;
    m->max_kt = m->max_kt_fused = m->max_qc = m->max_keys = 0;
    for (int i = 0; i < (int)items.size(); i++) {
        const auto& it = items[i];
        m->max_kt = std::max(m->max_kt, tiles(it));
        if (i >= n_long) m->max_kt_fused = std::max(m->max_kt_fused, tiles(it));
        m->max_qc = std::max(m->max_qc, it.q_count);
        m->max_keys = std::max(m->max_keys, it.pos0 + it.q_count);
    }
    // (query, key) pairs the items attend over, and those of the long items
    m->attn_pairs = m->attn_pairs_long = 0;
    for (int i = 0; i < (int)items.size(); i++) {
        const auto& it = items[i];
        const int64_t pairs = (int64_t)it.q_count * it.pos0 + (int64_t)it.q_count * (it.q_count + 1) / 2;
        m->attn_pairs += pairs;
        if (i < n_long) m->attn_pairs_long += pairs;
    }
    HIP_TRY(m->scores.ensure(sizeof(float) * (size_t)std::max<int64_t>(off + m->pm_floats, 1)));
    HIP_TRY(m->items.ensure(sizeof(AttnItem) * items.size()));
    HIP_TRY(upload(m, m->items.p, items.data(), sizeof(AttnItem) * items.size()));
    HIP_TRY(m->chunks.ensure(sizeof(AttnChunk) * std::max<size_t>(chunks.size(), 1)));
    HIP_TRY(upload(m, m->chunks.p, chunks.data(), sizeof(AttnChunk) * chunks.size()));
    m->n_chunks = (int)chunks.size();
    return SHS_OK;
}

}  // namespace

extern "C" shs_status shs_forward(shs_model* m, const int32_t* tokens, int32_t n, int32_t head_mode,
                                  const int32_t* vocab_ids, int32_t n_ids, float* logits_out,
                                  const volatile int32_t* cancel)
{
    if (!m || !tokens) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (n <= 0) return fail(SHS_E_INVALID_ARGUMENT, "No tokens to forward.");
    if (head_mode < 0 || head_mode > 2) return fail(SHS_E_INVALID_ARGUMENT, "head_mode must be 0, 1 or 2");
    if (head_mode == 1 && (!vocab_ids || n_ids <= 0 || !logits_out))
        return fail(SHS_E_INVALID_ARGUMENT, "selected-rows head needs vocab_ids and logits_out");
    if (head_mode == 2 && !logits_out) return fail(SHS_E_INVALID_ARGUMENT, "full head needs logits_out");
    const shs_config& c = m->cfg;
    shs_status st;
    if ((st = check_ids(tokens, n, c.vocab, "Token id")) != SHS_OK) return st;
    if (head_mode == 1 && (st = check_ids(vocab_ids, n_ids, c.vocab, "Row")) != SHS_OK) return st;
    HIP_TRY(hipSetDevice(m->device));
    const int start = m->len;
    if ((st = ensure_kv(m, start + n)) != SHS_OK) return st;
    if ((st = ensure_rope(m, start + n)) != SHS_OK) return st;
    if ((st = ensure_work(m, n)) != SHS_OK) return st;

    std::vector<int32_t> pos(n);
    for (int t = 0; t < n; t++) pos[t] = start + t;
    std::vector<AttnItem> items = causal_items(0, n, 0, start);
    HIP_TRY(begin_uploads(m));
    if ((st = place_items(m, items)) != SHS_OK) return st;
    HIP_TRY(upload(m, m->tokens.p, tokens, sizeof(int32_t) * n));
    HIP_TRY(upload(m, m->pos.p, pos.data(), sizeof(int32_t) * n));
    if (head_mode == 1) {
        HIP_TRY(m->ids.ensure(sizeof(int32_t) * n_ids));
        HIP_TRY(upload(m, m->ids.p, vocab_ids, sizeof(int32_t) * n_ids));
    }
    {
        Timed tm(m->prof, "embed", 0, m->stream);
        HIP_TRY(launch_embed(m->embd, m->tokens.as<int32_t>(), n, m->h.as<float>(), c.hidden, m->stream));
    }
    Capture cp{m, {}};
    if (m->cap_fn && cp.observe("embeddings", m->h.as<float>(), c.hidden, n, c.hidden) != SHS_OK) return SHS_E_DEVICE;

    st = run_layers(m, n, m->kc, m->vc, m->cap, start, 0, c.n_layer, m->items.as<AttnItem>(), (int)items.size(), cancel, true);
    if (st != SHS_OK) {
        (void)hipStreamSynchronize(m->stream);
        return st;
    }
    if (head_mode != 0) {
        int n_out = head_mode == 1 ? n_ids : c.vocab;
        HIP_TRY(m->logits.ensure(sizeof(float) * n_out));
        if ((st = run_head(m, {n - 1}, head_mode, m->ids.as<int32_t>(), n_ids, m->logits.as<float>())) != SHS_OK) return st;
        HIP_TRY(hipMemcpyAsync(logits_out, m->logits.p, sizeof(float) * n_out, hipMemcpyDeviceToHost, m->stream));
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (head_mode == 2 && m->cap_fn) m->cap_fn("logits", logits_out, 1, c.vocab, m->cap_user);
    // KvCache.Advance only after a complete pass (MinistralModel.cs:240).
    m->len = start + n;
    return SHS_OK;
}

extern "C" shs_status shs_forward_batch(shs_model* m, const int32_t* tokens, const int32_t* cu, int32_t n_seq,
                                        const int32_t* vocab_ids, int32_t n_ids, float* logits_out)
{
    if (!m || !tokens || !cu || !vocab_ids || !logits_out) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (n_seq <= 0 || n_ids <= 0) return fail(SHS_E_INVALID_ARGUMENT, "need at least one sequence and one vocab id");
    if (cu[0] != 0) return fail(SHS_E_INVALID_ARGUMENT, "cu_seqlens[0] must be 0");
    for (int s = 0; s < n_seq; s++)
        if (cu[s + 1] <= cu[s]) return fail(SHS_E_INVALID_ARGUMENT, "sequence %d is empty or cu_seqlens is not increasing", s);
    const int T = cu[n_seq];
    const shs_config& c = m->cfg;
    shs_status st;
    if ((st = check_ids(tokens, T, c.vocab, "Token id")) != SHS_OK) return st;
    if ((st = check_ids(vocab_ids, n_ids, c.vocab, "Row")) != SHS_OK) return st;
    HIP_TRY(hipSetDevice(m->device));
    int longest = 0;
    for (int s = 0; s < n_seq; s++) longest = std::max(longest, cu[s + 1] - cu[s]);
    if ((st = ensure_rope(m, longest)) != SHS_OK) return st;
    if ((st = ensure_work(m, T)) != SHS_OK) return st;
    // One layer's worth of packed K/V, reused layer after layer.
    const int cap = T;
    const size_t kvf = (size_t)c.n_kv_head * cap * c.head_dim;
    HIP_TRY(m->bkc.ensure(sizeof(float) * kvf));
    HIP_TRY(m->bvc.ensure(sizeof(float) * kvf));

    std::vector<int32_t> pos(T);
    std::vector<AttnItem> items;
    for (int s = 0; s < n_seq; s++) {
        for (int t = cu[s]; t < cu[s + 1]; t++) pos[t] = t - cu[s];
        auto v = causal_items(cu[s], cu[s + 1] - cu[s], cu[s], 0);
        items.insert(items.end(), v.begin(), v.end());
    }
    // The kernel takes items from the back: put the longest key ranges there.
    std::stable_sort(items.begin(), items.end(),
                     [](const AttnItem& x, const AttnItem& y) { return x.pos0 + x.q_count < y.pos0 + y.q_count; });
    HIP_TRY(begin_uploads(m));
    if ((st = place_items(m, items)) != SHS_OK) return st;
    HIP_TRY(m->ids.ensure(sizeof(int32_t) * n_ids));
    HIP_TRY(upload(m, m->tokens.p, tokens, sizeof(int32_t) * T));
    HIP_TRY(upload(m, m->pos.p, pos.data(), sizeof(int32_t) * T));
    HIP_TRY(upload(m, m->ids.p, vocab_ids, sizeof(int32_t) * n_ids));
    {
        Timed tm(m->prof, "embed", 0, m->stream);
        HIP_TRY(launch_embed(m->embd, m->tokens.as<int32_t>(), T, m->h.as<float>(), c.hidden, m->stream));
    }
    st = run_layers(m, T, m->bkc.as<float>(), m->bvc.as<float>(), cap, 0, 0, c.n_layer, m->items.as<AttnItem>(),
                    (int)items.size(), nullptr, false);
    if (st != SHS_OK) {
        (void)hipStreamSynchronize(m->stream);
        return st;
    }
    std::vector<int32_t> last(n_seq);
    for (int s = 0; s < n_seq; s++) last[s] = cu[s + 1] - 1;
    HIP_TRY(m->logits.ensure(sizeof(float) * (size_t)n_seq * n_ids));
    if ((st = run_head(m, last, 1, m->ids.as<int32_t>(), n_ids, m->logits.as<float>())) != SHS_OK) return st;
    HIP_TRY(hipMemcpyAsync(logits_out, m->logits.p, sizeof(float) * (size_t)n_seq * n_ids, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_layer_forward(shs_model* m, int32_t layer, const float* x, int32_t n, float* y)
{
    if (!m || !x || !y) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (layer < 0 || layer >= m->cfg.n_layer) return fail(SHS_E_OUT_OF_RANGE, "layer %d does not exist", layer);
    if (n <= 0) return fail(SHS_E_INVALID_ARGUMENT, "No tokens to forward.");
    const shs_config& c = m->cfg;
    HIP_TRY(hipSetDevice(m->device));
    shs_status st;
    if ((st = ensure_kv(m, n)) != SHS_OK) return st;
    if ((st = ensure_rope(m, n)) != SHS_OK) return st;
    if ((st = ensure_work(m, n)) != SHS_OK) return st;
    std::vector<int32_t> pos(n);
    for (int t = 0; t < n; t++) pos[t] = t;
    std::vector<AttnItem> items = causal_items(0, n, 0, 0);
    HIP_TRY(begin_uploads(m));
    if ((st = place_items(m, items)) != SHS_OK) return st;
    HIP_TRY(upload(m, m->pos.p, pos.data(), sizeof(int32_t) * n));
    HIP_TRY(hipMemcpyAsync(m->h.p, x, sizeof(float) * (size_t)n * c.hidden, hipMemcpyHostToDevice, m->stream));
    m->len = 0;
    st = run_layers(m, n, m->kc, m->vc, m->cap, 0, layer, layer + 1, m->items.as<AttnItem>(), (int)items.size(), nullptr, true);
    (void)hipStreamSynchronize(m->stream);
    if (st != SHS_OK) return st;
    HIP_TRY(hipMemcpy(y, m->h.p, sizeof(float) * (size_t)n * c.hidden, hipMemcpyDeviceToHost));
    m->len = 0;
    return SHS_OK;
}

extern "C" shs_status shs_synchronize(shs_model* m)
{
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null model");
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_debug_expf(const float* x, int32_t n, float* y, int32_t device)
{
    if (!x || !y || n < 0) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    shs_status st = select_device(device);
    if (st != SHS_OK) return st;
    float* d = nullptr;
    HIP_TRY(hipMalloc(&d, sizeof(float) * 2 * (size_t)std::max(n, 1)));
    hipError_t e = hipMemcpy(d, x, sizeof(float) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_expf(d, n, d + n, nullptr);
    if (e == hipSuccess) e = hipMemcpy(y, d + n, sizeof(float) * n, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return hip_fail(e, "shs_debug_expf");
    return SHS_OK;
}

// --------------------------------------------------------------- profiling

extern "C" shs_status shs_profile_enable(shs_model* m, int32_t enable)
{
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null model");
    m->prof.on = enable != 0;
    return SHS_OK;
}

extern "C" shs_status shs_profile_read(shs_model* m, const char* cls, int64_t* launches, double* total_ms, double* total_ops)
{
    if (!m || !cls) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    (void)hipSetDevice(m->device);
    m->prof.collect();
    // "name" reads one class; "prefix*" sums every class that starts with prefix.
    std::string key(cls);
    const bool prefix = !key.empty() && key.back() == '*';
    if (prefix) key.pop_back();
    int64_t n = 0;
    double ms = 0, ops = 0;
    for (const auto& kv : m->prof.totals) {
        if (prefix ? kv.first.compare(0, key.size(), key) != 0 : kv.first != key) continue;
        n += kv.second.first;
        ms += kv.second.second.first;
        ops += kv.second.second.second;
    }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    if (total_ops) *total_ops = ops;
    return SHS_OK;
}

extern "C" shs_status shs_profile_reset(shs_model* m)
{
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null model");
    (void)hipSetDevice(m->device);
    m->prof.collect();
    m->prof.totals.clear();
    return SHS_OK;
}

// ------------------------------------------------------- quantized matmul

extern "C" shs_status shs_matrix_create(int32_t type, int32_t rows, int32_t cols, const void* data, int32_t device,
                                        shs_matrix** out)
{
    if (!data || !out) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (!type_supported(type))
        return fail(SHS_E_NOT_SUPPORTED, "%s has no integer GEMM kernel.", type_name(type));
    if (rows <= 0 || cols <= 0 || cols % 32)
        return fail(SHS_E_INVALID_ARGUMENT, "a %d x %d matrix: rows must be positive and cols a positive multiple of 32",
                    rows, cols);
    shs_status st = select_device(device);
    if (st != SHS_OK) return st;
    shs_matrix* m = new shs_matrix();
    m->device = device;
    hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = alloc_matrix(m->w, type, rows, cols, m->stream);
    Buf staging;
    if (e == hipSuccess) e = upload_rows(m->w, host_src(data), 0, rows, staging, m->stream);
    if (e != hipSuccess) {
        shs_matrix_free(m);
        return hip_fail(e, "shs_matrix_create");
    }
    *out = m;
    return SHS_OK;
}

extern "C" void shs_matrix_free(shs_matrix* m)
{
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    free_matrix(m->w);
    hipStream_t s = m->stream;
    delete m;
    if (s) (void)hipStreamDestroy(s);
}

static shs_status matmul_common(shs_matrix* m, const float* x, int T, int semantics, ActQ8* a, bool x_on_device)
{
    if (!m || !x) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (T <= 0) return fail(SHS_E_INVALID_ARGUMENT, "tokens must be positive");
    if (semantics != 0 && semantics != 1) return fail(SHS_E_INVALID_ARGUMENT, "semantics must be 0 or 1");
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(m->act.ensure(T, m->w.cols, a));
    const float* xd = x;
    if (!x_on_device) {
        HIP_TRY(m->x.ensure(sizeof(float) * (size_t)T * m->w.cols));
        HIP_TRY(hipMemcpyAsync(m->x.p, x, sizeof(float) * (size_t)T * m->w.cols, hipMemcpyHostToDevice, m->stream));
        xd = m->x.as<float>();
    }
    HIP_TRY(launch_quant_act(xd, m->w.cols, *a, semantics, m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_matmul(shs_matrix* m, const float* x, int32_t T, float* y, int32_t semantics)
{
    if (!y) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    ActQ8 a;
    shs_status st = matmul_common(m, x, T, semantics, &a, false);
    if (st != SHS_OK) return st;
    HIP_TRY(m->y.ensure(sizeof(float) * (size_t)T * m->w.rows));
    HIP_TRY(launch_gemm(m->w, a, m->y.as<float>(), m->w.rows, GEMM_STORE, m->stream));
    HIP_TRY(hipMemcpyAsync(y, m->y.p, sizeof(float) * (size_t)T * m->w.rows, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_matmul_rows(shs_matrix* m, const int32_t* ids, int32_t n_ids, const float* x, int32_t T, float* y)
{
    if (!ids || !y || n_ids <= 0) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (!m) return fail(SHS_E_INVALID_ARGUMENT, "null matrix");
    for (int i = 0; i < n_ids; i++)
        if (ids[i] < 0 || ids[i] >= m->w.rows)
            return fail(SHS_E_OUT_OF_RANGE, "Row %d is outside the matrix's %d rows.", ids[i], m->w.rows);
    ActQ8 a;
    shs_status st = matmul_common(m, x, T, 0, &a, false);
    if (st != SHS_OK) return st;
    HIP_TRY(m->ids.ensure(sizeof(int32_t) * n_ids));
    HIP_TRY(m->y.ensure(sizeof(float) * (size_t)T * n_ids));
    HIP_TRY(hipMemcpyAsync(m->ids.p, ids, sizeof(int32_t) * n_ids, hipMemcpyHostToDevice, m->stream));
    HIP_TRY(launch_gemv_rows(m->w, a, m->ids.as<int32_t>(), n_ids, m->y.as<float>(), m->stream));
    HIP_TRY(hipMemcpyAsync(y, m->y.p, sizeof(float) * (size_t)T * n_ids, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_matmul_block_sums(shs_matrix* m, const float* x, int32_t T, int32_t* out)
{
    if (!out) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    ActQ8 a;
    shs_status st = matmul_common(m, x, T, 0, &a, false);
    if (st != SHS_OK) return st;
    size_t n = (size_t)T * m->w.rows * m->w.blocks;
    HIP_TRY(m->sums.ensure(sizeof(int32_t) * n));
    HIP_TRY(launch_gemm_block_sums(m->w, a, m->sums.as<int32_t>(), m->stream));
    HIP_TRY(hipMemcpyAsync(out, m->sums.p, sizeof(int32_t) * n, hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

extern "C" shs_status shs_matmul_device(shs_matrix* m, const float* x_dev, int32_t T, float* y_dev)
{
    if (!y_dev) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    ActQ8 a;
    shs_status st = matmul_common(m, x_dev, T, 0, &a, true);
    if (st != SHS_OK) return st;
    HIP_TRY(launch_gemm(m->w, a, y_dev, m->w.rows, GEMM_STORE, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

// shs_matmul_device with the activation codes in the library's fixed per-GPU scratch
// (noalloc_scratch): no hipMalloc, hipFree or allocating library call on any path.
extern "C" shs_status shs_matmul_device_noalloc(shs_matrix* m, const float* x_dev, int32_t T, float* y_dev)
{
    if (!m || !x_dev || !y_dev) return fail(SHS_E_INVALID_ARGUMENT, "null argument");
    if (T <= 0) return fail(SHS_E_INVALID_ARGUMENT, "tokens must be positive");
    const int K = m->w.cols;
    const size_t need = act_q8_bytes(T, K);
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(SHS_E_OUT_OF_RANGE,
                    "%d tokens of %d columns need %zu bytes of activation scratch; shs_matmul_device_noalloc holds "
                    "at most %zu (about %zu tokens at this width). Split the call or use shs_matmul_device.",
                    T, K, need, NOALLOC_SCRATCH_BYTES, NOALLOC_SCRATCH_BYTES / ((size_t)K + (size_t)K / 2));
    HIP_TRY(hipSetDevice(m->device));
    uint8_t* base = nullptr;
    HIP_TRY(noalloc_scratch(m->device, &base));
    ActQ8 a = act_q8_view(base, T, K);
    // k_quant_act writes every code, scale and column up to Tpad (zeros past T), so nothing
    // left by an earlier call is read.
    HIP_TRY(launch_quant_act(x_dev, K, a, 0, m->stream));
    HIP_TRY(launch_gemm(m->w, a, y_dev, m->w.rows, GEMM_STORE, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return SHS_OK;
}

// Error hook for the GGUF reader (shs_gguf.cpp), which shares this thread-local message.
extern "C" __attribute__((visibility("hidden"))) shs_status shs_gguf_fail(shs_status code, const char* msg)
{
    g_error = msg;
    return code;
}
