// .qora v1 reader and writer (save.rs:1-262), all little-endian,
// length-prefixed:
//   "QOR3", u32 version = 1, u8 format (0 = F16, 1 = Q4)
//   u32 num_layers, vocab, hidden, rope_half_dim; u64 len + u8[] use-RoPE flags
//   per layer: 7 weights q,k,v,o,gate,up,down, each u64 k, u64 n then
//     F16: u64 len + f16[]   |   Q4: u64 len + u8[] packed, u64 len + f16[] scales
//   then u64 len + f16[] input norm, u64 len + f16[] post-attention norm,
//   u32 num_heads, num_kv_heads, head_dim, num_kv_groups
//   embedding weight (k = vocab, n = hidden), u64 len + f16[] final norm,
//   u64 len + f32[] rope_cos, u64 len + f32[] rope_sin
// The reader streams the file and uploads each weight as it is read, so the
// host never holds the whole model.
#include "../../include/qora_hip.h"

#include <cstdio>
#include <new>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct Reader {
    FILE* f = nullptr;
    bool ok = true;
    uint64_t left = 0;   // bytes not yet read
    explicit Reader(const char* path) : f(std::fopen(path, "rb")) {
        ok = f != nullptr;
        if (ok && std::fseek(f, 0, SEEK_END) == 0) {
            const long end = std::ftell(f);
            ok = end >= 0 && std::fseek(f, 0, SEEK_SET) == 0;
            left = ok ? (uint64_t)end : 0;
        } else {
            ok = false;
        }
    }
    ~Reader() { if (f) std::fclose(f); }
    bool bytes(void* dst, size_t n) {
        if (!ok) return false;
        if (n > left || (n && std::fread(dst, 1, n, f) != n)) ok = false;
        else left -= n;
        return ok;
    }
    uint32_t u32() { uint8_t b[4] = {0}; bytes(b, 4); return (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24; }
    uint64_t u64() { const uint64_t lo = u32(); const uint64_t hi = u32(); return lo | hi << 32; }
    uint8_t u8() { uint8_t b = 0; bytes(&b, 1); return b; }
    // length-prefixed vector of `elem`-byte items, bounded by `max_len` and by
    // the bytes left in the file (a corrupt length fails before any allocation)
    template <class T>
    bool vec(std::vector<T>& out, uint64_t max_len) {
        const uint64_t len = u64();
        if (!ok || len > max_len || len > left / sizeof(T)) { ok = false; return false; }
        out.resize(len);
        return bytes(out.data(), len * sizeof(T));
    }
};

struct Writer {
    FILE* f = nullptr;
    bool ok = true;
    explicit Writer(const char* path) : f(std::fopen(path, "wb")) { ok = f != nullptr; }
    ~Writer() { if (f) std::fclose(f); }
    void bytes(const void* src, size_t n) { if (ok && n && std::fwrite(src, 1, n, f) != n) ok = false; }
    void u32(uint32_t v) { const uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)}; bytes(b, 4); }
    void u64(uint64_t v) { u32((uint32_t)v); u32((uint32_t)(v >> 32)); }
    void u8(uint8_t v) { bytes(&v, 1); }
    void vec(const void* data, uint64_t len, size_t elem) { u64(len); bytes(data, len * elem); }
};

constexpr uint64_t kMaxElems = 1ull << 36;

int read_weight(qora_hip_ctx* ctx, Reader& r, uint8_t fmt, uint64_t* k, uint64_t* n, uint32_t* wid) {
    *k = r.u64();
    *n = r.u64();
    if (!r.ok) return QORA_HIP_E_IO;
    if (fmt == 0) {
        std::vector<uint16_t> d;
        if (!r.vec(d, kMaxElems)) return QORA_HIP_E_IO;
        return qora_hip_upload_f16(ctx, d.data(), d.size(), *k, *n, wid);
    }
    std::vector<uint8_t> p;
    std::vector<uint16_t> s;
    if (!r.vec(p, kMaxElems) || !r.vec(s, kMaxElems)) return QORA_HIP_E_IO;
    return qora_hip_upload_q4(ctx, p.data(), p.size(), s.data(), s.size(), *k, *n, wid);
}

// Uploads of one load, released again if the load fails.
struct Uploads {
    qora_hip_ctx* ctx;
    std::vector<uint32_t> wids;
    bool keep = false;
    ~Uploads() {
        if (!keep)
            for (uint32_t w : wids) (void)qora_hip_release_weight(ctx, w);
    }
};

int load_model(qora_hip_ctx* ctx, const char* path, uint32_t kv_capacity, uint32_t kv_dtype, Uploads& up) {
    Reader r(path);
    if (!r.ok) return QORA_HIP_E_IO;
    char magic[4];
    if (!r.bytes(magic, 4) || std::memcmp(magic, "QOR3", 4) != 0) return QORA_HIP_E_IO;   // save.rs:160-162
    const uint32_t version = r.u32();
    if (!r.ok || version != 1) return QORA_HIP_E_IO;                                         // save.rs:163-169
    const uint8_t fmt = r.u8();
    if (!r.ok || fmt > 1) return QORA_HIP_E_IO;                                              // save.rs:233-236
    const uint32_t num_layers = r.u32(), vocab = r.u32(), hidden = r.u32(), half = r.u32();
    std::vector<uint8_t> flags;
    if (!r.vec(flags, 1u << 20)) return QORA_HIP_E_IO;
    for (uint8_t& b : flags) b = b != 0;   // read_bool_vec: b != 0 (save.rs:107-112)
    if (flags.size() < num_layers) return QORA_HIP_E_IO;

    std::vector<uint32_t> wids((size_t)num_layers * 7);
    std::vector<std::vector<uint16_t>> in_norm(num_layers), post_norm(num_layers);
    uint32_t heads = 0, kv_heads = 0, head_dim = 0, groups = 0;
    uint64_t inter = 0;
    for (uint32_t l = 0; l < num_layers; ++l) {
        for (int j = 0; j < 7; ++j) {
            uint64_t k, n;
            if (int rc = read_weight(ctx, r, fmt, &k, &n, &wids[(size_t)l * 7 + j])) return rc;
            up.wids.push_back(wids[(size_t)l * 7 + j]);
            if (j == 4) inter = n;
        }
        if (!r.vec(in_norm[l], kMaxElems) || !r.vec(post_norm[l], kMaxElems)) return QORA_HIP_E_IO;
        if (in_norm[l].size() != hidden || post_norm[l].size() != hidden) return QORA_HIP_E_IO;
        const uint32_t h = r.u32(), kvh = r.u32(), hd = r.u32(), g = r.u32();
        if (!r.ok) return QORA_HIP_E_IO;
        if (l == 0) { heads = h; kv_heads = kvh; head_dim = hd; groups = g; }
        else if (h != heads || kvh != kv_heads || hd != head_dim || g != groups) return QORA_HIP_E_INVALID;
    }
    uint64_t ek, en;
    uint32_t embed_wid;
    if (int rc = read_weight(ctx, r, fmt, &ek, &en, &embed_wid)) return rc;
    up.wids.push_back(embed_wid);
    std::vector<uint16_t> final_norm;
    std::vector<float> cos_t, sin_t;
    if (!r.vec(final_norm, kMaxElems) || !r.vec(cos_t, kMaxElems) || !r.vec(sin_t, kMaxElems)) return QORA_HIP_E_IO;
    if (final_norm.size() != hidden || cos_t.size() != sin_t.size()) return QORA_HIP_E_IO;

    std::vector<const uint16_t*> inp(num_layers), post(num_layers);
    for (uint32_t l = 0; l < num_layers; ++l) { inp[l] = in_norm[l].data(); post[l] = post_norm[l].data(); }
    qora_model_desc d{};
    d.num_layers = num_layers;
    d.vocab = vocab;
    d.hidden = hidden;
    d.intermediate = (uint32_t)inter;
    d.num_heads = heads;
    d.num_kv_heads = kv_heads;
    d.head_dim = head_dim;
    d.num_kv_groups = groups;
    d.rope_half_dim = half;
    d.format = fmt;
    d.layer_wids = wids.data();
    d.input_norm = inp.data();
    d.post_attn_norm = post.data();
    d.embed_wid = embed_wid;
    d.final_norm = final_norm.data();
    d.rope_cos = cos_t.data();
    d.rope_sin = sin_t.data();
    d.rope_positions = half ? cos_t.size() / half : 0;
    d.use_rope = flags.data();
    d.kv_capacity = kv_capacity;
    d.kv_dtype = kv_dtype;
    const int rc = qora_hip_model_init(ctx, &d);
    up.keep = rc == QORA_HIP_OK;
    return rc;
}

}  // namespace

extern "C" int qora_hip_load_model(qora_hip_ctx* ctx, const char* path, uint32_t kv_capacity, uint32_t kv_dtype) {
    if (!ctx || !path) return QORA_HIP_E_INVALID;
    // no exception crosses the C ABI (a Rust caller would abort)
    try {
        Uploads up{ctx, {}, false};
        return load_model(ctx, path, kv_capacity, kv_dtype, up);
    } catch (const std::bad_alloc&) {
        return QORA_HIP_E_NOMEM;
    } catch (...) {
        return QORA_HIP_E_IO;
    }
}

extern "C" int qora_file_write(const char* path, const qora_host_model* m) {
    if (!path || !m || m->format > 1) return QORA_HIP_E_INVALID;
    Writer w(path);
    if (!w.ok) return QORA_HIP_E_IO;
    const uint64_t H = m->hidden, I = m->intermediate;
    const uint64_t qd = (uint64_t)m->num_heads * m->head_dim, kvd = (uint64_t)m->num_kv_heads * m->head_dim;
    const uint64_t shapes[7][2] = {{H, qd}, {H, kvd}, {H, kvd}, {qd, H}, {H, I}, {H, I}, {I, H}};
    auto put_weight = [&](const void* data, const uint16_t* scales, uint64_t k, uint64_t n) {
        w.u64(k);
        w.u64(n);
        if (m->format == 0) {
            w.vec(data, k * n, 2);
        } else {
            w.vec(data, k * n / 2, 1);
            w.vec(scales, k * n / 32, 2);
        }
    };
    w.bytes("QOR3", 4);
    w.u32(1);
    w.u8((uint8_t)m->format);
    w.u32(m->num_layers);
    w.u32(m->vocab);
    w.u32(m->hidden);
    w.u32(m->rope_half_dim);
    w.u64(m->num_layers);
    for (uint32_t l = 0; l < m->num_layers; ++l) w.u8(m->use_rope[l] ? 1 : 0);
    for (uint32_t l = 0; l < m->num_layers; ++l) {
        for (int j = 0; j < 7; ++j)
            put_weight(m->w_data[(size_t)l * 7 + j], m->w_scales ? m->w_scales[(size_t)l * 7 + j] : nullptr,
                       shapes[j][0], shapes[j][1]);
        w.vec(m->input_norm[l], H, 2);
        w.vec(m->post_attn_norm[l], H, 2);
        w.u32(m->num_heads);
        w.u32(m->num_kv_heads);
        w.u32(m->head_dim);
        w.u32(m->num_kv_groups);
    }
    put_weight(m->embed_data, m->embed_scales, m->vocab, H);
    w.vec(m->final_norm, H, 2);
    w.vec(m->rope_cos, m->rope_positions * m->rope_half_dim, 4);
    w.vec(m->rope_sin, m->rope_positions * m->rope_half_dim, 4);
    return w.ok ? QORA_HIP_OK : QORA_HIP_E_IO;
}
