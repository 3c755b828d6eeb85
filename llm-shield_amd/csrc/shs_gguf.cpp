// shs_open: GGUF v2/v3 reader in front of shs_open_tensors.
//
// Follows GgufFile (GgufFile.cs:76-199) for the container — header, typed metadata,
// tensor table, general.alignment (default 32), truncation check — and
// ModelConfig.FromGguf (ModelConfig.cs:62-112) for the hyperparameters and their
// defaults. The file is memory-mapped read-only and unmapped before returning.
#include "shieldstral_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

extern "C" __attribute__((visibility("hidden"))) shs_status shs_gguf_fail(shs_status code, const char* msg);

namespace {

enum GType { U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7, STR = 8, ARR = 9, U64 = 10, I64 = 11, F64 = 12 };

struct Value {
    int type = -1;
    double num = 0;          // numeric scalar
    std::string str;         // string scalar
    uint64_t arr_len = 0;    // array length
};

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    bool ok = true;
    // pos <= n always holds, so n - pos cannot wrap; pos + k could (a 64-bit string
    // length near 2^64 from a damaged header).
    bool need(uint64_t k)
    {
        if (!ok || k > n - pos) ok = false;
        return ok;
    }
    template <class T> T get()
    {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str()
    {
        uint64_t len = get<uint64_t>();
        if (!need(len)) return {};
        std::string s(reinterpret_cast<const char*>(p + pos), len);
        pos += len;
        return s;
    }
    bool skip_scalar(uint32_t t)
    {
        static const int size[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (t == STR) { str(); return ok; }
        if (t > F64 || t == ARR) { ok = false; return false; }
        return need(size[t]) && (pos += size[t], true);
    }
    Value value(uint32_t t)
    {
        Value v;
        v.type = (int)t;
        switch (t) {
        case U8: v.num = get<uint8_t>(); break;
        case I8: v.num = get<int8_t>(); break;
        case U16: v.num = get<uint16_t>(); break;
        case I16: v.num = get<int16_t>(); break;
        case U32: v.num = get<uint32_t>(); break;
        case I32: v.num = get<int32_t>(); break;
        case F32: v.num = get<float>(); break;
        case BOOL: v.num = get<uint8_t>(); break;
        case STR: v.str = str(); break;
        case U64: v.num = (double)get<uint64_t>(); break;
        case I64: v.num = (double)get<int64_t>(); break;
        case F64: v.num = get<double>(); break;
        case ARR: {
            uint32_t et = get<uint32_t>();
            v.arr_len = get<uint64_t>();
            for (uint64_t i = 0; i < v.arr_len && ok; i++) skip_scalar(et);
            break;
        }
        default: ok = false;
        }
        return v;
    }
};

struct Mapping {
    void* base = MAP_FAILED;
    size_t size = 0;
    ~Mapping()
    {
        if (base != MAP_FAILED) munmap(base, size);
    }
};

shs_status err(shs_status code, const char* fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return shs_gguf_fail(code, buf);
}

}  // namespace

// Reads the file's header and ModelConfig; with out == nullptr it stops there (after
// the truncation check, as GgufFile's constructor runs it before FromGguf) and reports
// the config through cfg_out, else it uploads the tensors.
static shs_status open_gguf(const char* path, int32_t device, int32_t initial_capacity, shs_model** out,
                            shs_config* cfg_out)
{
    if (!path || (!out && !cfg_out)) return err(SHS_E_INVALID_ARGUMENT, "null argument");
    if (out) *out = nullptr;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return err(SHS_E_IO, "%s: cannot open (%s)", path, strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return err(SHS_E_IO, "%s: cannot stat", path);
    }
    Mapping map;
    map.size = (size_t)sb.st_size;
    if (map.size > 0) map.base = mmap(nullptr, map.size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map.size < 24 || map.base == MAP_FAILED)
        return err(SHS_E_INVALID_DATA, "%s is not a GGUF file (too short to hold a header); re-download it", path);
    Reader r{static_cast<const uint8_t*>(map.base), map.size};
    uint32_t magic = r.get<uint32_t>();
    if (magic != 0x46554747u) return err(SHS_E_INVALID_DATA, "%s is not a GGUF file (bad magic); re-download it", path);
    uint32_t version = r.get<uint32_t>();
    if (version < 2 || version > 3) return err(SHS_E_NOT_SUPPORTED, "%s is GGUF version %u; versions 2 and 3 are read", path, version);
    uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    std::map<std::string, Value> kv;
    for (uint64_t i = 0; i < n_kv && r.ok; i++) {
        std::string key = r.str();
        uint32_t t = r.get<uint32_t>();
        kv[key] = r.value(t);
    }
    struct TI { std::string name; uint32_t type; std::vector<uint64_t> dims; uint64_t offset; };
    std::vector<TI> infos;
    for (uint64_t i = 0; i < n_tensors && r.ok; i++) {
        TI ti;
        ti.name = r.str();
        uint32_t nd = r.get<uint32_t>();
        if (nd > 4) { r.ok = false; break; }
        for (uint32_t d = 0; d < nd; d++) ti.dims.push_back(r.get<uint64_t>());
        ti.type = r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        infos.push_back(ti);
    }
    if (!r.ok) return err(SHS_E_IO, "%s is truncated inside its header; re-download it", path);
    uint64_t align = 32;
    auto ai = kv.find("general.alignment");
    if (ai != kv.end()) {
        double v = ai->second.num;
        bool numeric = ai->second.type != STR && ai->second.type != ARR;
        if (!numeric || !(v >= 1.0) || v > (double)map.size || v != (double)(uint64_t)v)
            return err(SHS_E_INVALID_DATA, "%s has general.alignment %g; it must be a whole number from 1 to the file "
                                           "size. Re-download the file.", path, v);
        align = (uint64_t)v;
    }
    // r.pos <= map.size and align <= map.size, so neither the sum nor the product wraps.
    uint64_t data_off = (r.pos + align - 1) / align * align;
    if (data_off > map.size)
        return err(SHS_E_IO, "%s is truncated: its tensor data would start past the end of the file; re-download it",
                   path);

    auto num = [&](const std::string& k, double dflt, bool* found = nullptr) {
        auto it = kv.find(k);
        bool f = it != kv.end() && it->second.type != STR && it->second.type != ARR;
        if (found) *found = f;
        return f ? it->second.num : dflt;
    };
    auto str = [&](const std::string& k) {
        auto it = kv.find(k);
        return (it != kv.end() && it->second.type == STR) ? it->second.str : std::string();
    };
    std::string arch = str("general.architecture");
    if (arch.empty()) return err(SHS_E_INVALID_DATA, "%s has no general.architecture.", path);
    if (arch != "mistral3" && arch != "ministral3" && arch != "llama")
        return err(SHS_E_NOT_SUPPORTED, "%s is architecture '%s'; this runtime implements the Ministral-3 backbone "
                                        "that Shieldstral uses (GGUF architecture \"mistral3\").", path, arch.c_str());
    const std::string a = arch + ".";
    bool found = false;
    shs_config c{};
    snprintf(c.architecture, sizeof c.architecture, "%s", arch.c_str());
    c.n_head = (int)num(a + "attention.head_count", 0, &found);
    if (!found) return err(SHS_E_KEY_NOT_FOUND, "%s has no %sattention.head_count", path, a.c_str());
    c.hidden = (int)num(a + "embedding_length", 0, &found);
    if (!found) return err(SHS_E_KEY_NOT_FOUND, "%s has no %sembedding_length", path, a.c_str());
    c.head_dim = (int)num(a + "attention.key_length", c.hidden / (c.n_head > 0 ? c.n_head : 1));
    c.n_layer = (int)num(a + "block_count", 0, &found);
    if (!found) return err(SHS_E_KEY_NOT_FOUND, "%s has no %sblock_count", path, a.c_str());
    c.n_kv_head = (int)num(a + "attention.head_count_kv", c.n_head);
    c.ffn = (int)num(a + "feed_forward_length", 0, &found);
    if (!found) return err(SHS_E_KEY_NOT_FOUND, "%s has no %sfeed_forward_length", path, a.c_str());
    auto tok = kv.find("tokenizer.ggml.tokens");
    c.vocab = (tok != kv.end() && tok->second.type == ARR) ? (int)tok->second.arr_len : (int)num(a + "vocab_size", 0);
    c.rms_eps = (float)num(a + "attention.layer_norm_rms_epsilon", 1e-5);
    c.rope_theta = (float)num(a + "rope.freq_base", 10000.0);
    c.rope_dim = (int)num(a + "rope.dimension_count", c.head_dim);
    c.rope_scale = (float)num(a + "rope.scaling.factor", 1.0);
    std::string rtype = str(a + "rope.scaling.type");
    c.rope_orig_ctx = (int)num(a + "rope.scaling.original_context_length", 0);
    c.yarn_beta_fast = (float)num(a + "rope.scaling.yarn_beta_fast", num(a + "rope.scaling.beta_fast", 32.0));
    c.yarn_beta_slow = (float)num(a + "rope.scaling.yarn_beta_slow", num(a + "rope.scaling.beta_slow", 1.0));
    c.yarn_ext_factor = (float)num(a + "rope.scaling.yarn_ext_factor", 1.0);
    c.yarn_mscale = (float)num(a + "rope.scaling.mscale", 0.0);
    c.yarn_mscale_all_dim = (float)num(a + "rope.scaling.yarn_log_multiplier", num(a + "rope.scaling.mscale_all_dim", 0.0));
    c.rope_attn_factor = (float)num(a + "rope.scaling.attn_factor", num(a + "rope.scaling.yarn_attn_factor", 1.0));
    c.attn_temperature = (float)num(a + "attention.temperature_scale", num(a + "rope.scaling_beta", 0.0));
    c.yarn_active = (rtype == "yarn" && c.rope_orig_ctx > 0 && c.yarn_ext_factor != 0.0f && c.rope_scale > 1.0f) ? 1 : 0;
    if (c.n_kv_head <= 0 || c.n_head % c.n_kv_head != 0)
        return err(SHS_E_INVALID_DATA, "%d attention heads do not divide into %d KV heads.", c.n_head, c.n_kv_head);

    // Tensor table → shs_tensor, with GgufFile's truncation check (GgufFile.cs:156-172).
    // Byte size of n elements, or false for a type this reader does not size (the
    // reference skips those too) or a size that does not fit 64 bits.
    auto type_bytes = [](uint32_t t, uint64_t n, uint64_t* out) -> bool {
        uint64_t per, group;
        switch (t) {
        case 0: per = 4; group = 1; break;
        case 1: per = 2; group = 1; break;
        case 2: per = 18; group = 32; break;
        case 3: per = 20; group = 32; break;
        case 6: per = 22; group = 32; break;
        case 7: per = 24; group = 32; break;
        case 8: per = 34; group = 32; break;
        default: return false;
        }
        return !__builtin_mul_overflow(n / group, per, out);
    };
    const uint64_t room = map.size - data_off;  // bytes from the data section to the end
    std::vector<shs_tensor> ts;
    ts.reserve(infos.size());
    for (auto& ti : infos) {
        uint64_t count = 1;
        bool huge = false;
        for (auto d : ti.dims) huge |= __builtin_mul_overflow(count, d, &count);
        if (huge || ti.offset > room)
            return err(SHS_E_IO, "%s is truncated or damaged: tensor '%s' starts past the end of the file; "
                                 "re-download it", path, ti.name.c_str());
        uint64_t bytes = 0;
        if (type_bytes(ti.type, count, &bytes) && bytes > room - ti.offset)
            return err(SHS_E_IO, "%s is truncated: tensor '%s' ends past the end of the file; re-download it", path,
                       ti.name.c_str());
        shs_tensor t{};
        t.name = ti.name.c_str();
        t.type = (int32_t)ti.type;
        t.ne0 = ti.dims.size() > 0 ? (int64_t)ti.dims[0] : 1;
        t.ne1 = ti.dims.size() > 1 ? (int64_t)ti.dims[1] : 1;
        t.data = static_cast<const uint8_t*>(map.base) + data_off + ti.offset;
        ts.push_back(t);
    }
    if (!out) {
        *cfg_out = c;
        return SHS_OK;
    }
    return shs_open_tensors(&c, ts.data(), (int32_t)ts.size(), device, initial_capacity, out);
}

// No C++ exception may cross the C ABI: an allocation that fails while the header is
// parsed becomes a status.
static shs_status guarded(const char* path, int32_t device, int32_t initial_capacity, shs_model** out,
                          shs_config* cfg_out)
{
    try {
        return open_gguf(path, device, initial_capacity, out, cfg_out);
    } catch (const std::bad_alloc&) {
        return err(SHS_E_IO, "%s: out of host memory while reading its header", path ? path : "(null)");
    } catch (...) {
        return err(SHS_E_INVALID_DATA, "%s: its header could not be read; re-download it", path ? path : "(null)");
    }
}

extern "C" shs_status shs_open(const char* path, int32_t device, int32_t initial_capacity, shs_model** out)
{
    if (!out) return err(SHS_E_INVALID_ARGUMENT, "null argument");
    return guarded(path, device, initial_capacity, out, nullptr);
}

extern "C" shs_status shs_read_config(const char* path, shs_config* out)
{
    if (!out) return err(SHS_E_INVALID_ARGUMENT, "null argument");
    return guarded(path, 0, 0, nullptr, out);
}
