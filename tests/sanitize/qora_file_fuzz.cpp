// The .qora v1 reader (qora-llm_amd/csrc/qora_file.cpp, save.rs:154-262) and
// the synthetic generator (csrc/synth.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer, on the CPU.
//
// The reader hands each weight to the device upload API; here that API is a
// host-only recorder (below) that checks the sizes the real one checks and
// copies every byte it is given, so the sanitizers see each read. The test:
//   1. a valid small model (Q4 and F16) written by qora_file_write loads, and
//      the recorded weights equal the written ones byte for byte;
//   2. the file truncated at every length up to 512 bytes and at a stride
//      through the rest is refused, with every upload of the failed load
//      released;
//   3. seeded random byte and bit corruptions, and 8-byte runs of 0xFF
//      (huge length fields) at every offset of the header and first layer,
//      load or are refused without a sanitizer report, and a refused load
//      leaves no upload alive.
// Exit status 0 when every case holds.
#include "../../include/qora_hip.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

struct Upload {
    bool alive;
    bool q4;
    uint64_t k, n;
    std::vector<uint8_t> a;
    std::vector<uint16_t> b;
};

struct qora_hip_ctx {
    std::vector<Upload> w;
    bool model = false;
    uint32_t model_layers = 0;
};

extern "C" int qora_hip_upload_q4(qora_hip_ctx* c, const uint8_t* packed, size_t packed_len, const uint16_t* scales,
                                  size_t scales_len, uint64_t k, uint64_t n, uint32_t* wid) {
    if (!c || !packed || !scales || !wid) return QORA_HIP_E_INVALID;
    if (k == 0 || n == 0 || n % 32 != 0 || packed_len != k * n / 2 || scales_len != k * n / 32)
        return QORA_HIP_E_INVALID;
    Upload u{true, true, k, n, std::vector<uint8_t>(packed, packed + packed_len),
             std::vector<uint16_t>(scales, scales + scales_len)};
    c->w.push_back(std::move(u));
    *wid = (uint32_t)(c->w.size() - 1);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_upload_f16(qora_hip_ctx* c, const uint16_t* data, size_t len, uint64_t k, uint64_t n,
                                   uint32_t* wid) {
    if (!c || !data || !wid) return QORA_HIP_E_INVALID;
    if (k == 0 || n == 0 || len != k * n) return QORA_HIP_E_INVALID;
    Upload u{true, false, k, n, {}, std::vector<uint16_t>(data, data + len)};
    c->w.push_back(std::move(u));
    *wid = (uint32_t)(c->w.size() - 1);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_release_weight(qora_hip_ctx* c, uint32_t wid) {
    if (!c || wid >= c->w.size() || !c->w[wid].alive) return QORA_HIP_E_INVALID;
    c->w[wid].alive = false;
    c->w[wid].a.clear();
    c->w[wid].b.clear();
    return QORA_HIP_OK;
}

// The checks of qora_hip_model_init that concern the description itself,
// reading every array it points to (shapes against the uploads).
extern "C" int qora_hip_model_init(qora_hip_ctx* c, const qora_model_desc* d) {
    if (!c || !d || !d->layer_wids || !d->input_norm || !d->post_attn_norm || !d->final_norm || !d->use_rope)
        return QORA_HIP_E_INVALID;
    if (d->num_layers == 0 || d->hidden == 0 || d->num_heads == 0 || d->num_kv_heads == 0 || d->head_dim == 0 ||
        d->intermediate == 0 || d->vocab == 0)
        return QORA_HIP_E_INVALID;
    const uint64_t qd = (uint64_t)d->num_heads * d->head_dim, kvd = (uint64_t)d->num_kv_heads * d->head_dim;
    const uint64_t H = d->hidden, I = d->intermediate;
    const uint64_t shapes[7][2] = {{H, qd}, {H, kvd}, {H, kvd}, {qd, H}, {H, I}, {H, I}, {I, H}};
    uint64_t sum = 0;
    for (uint32_t l = 0; l < d->num_layers; ++l) {
        for (int j = 0; j < 7; ++j) {
            const uint32_t wid = d->layer_wids[(size_t)l * 7 + j];
            if (wid >= c->w.size() || !c->w[wid].alive) return QORA_HIP_E_INVALID;
            if (c->w[wid].k != shapes[j][0] || c->w[wid].n != shapes[j][1]) return QORA_HIP_E_INVALID;
        }
        for (uint64_t i = 0; i < H; ++i) sum += d->input_norm[l][i] + d->post_attn_norm[l][i];
        sum += d->use_rope[l];
    }
    if (d->embed_wid >= c->w.size() || !c->w[d->embed_wid].alive) return QORA_HIP_E_INVALID;
    for (uint64_t i = 0; i < H; ++i) sum += d->final_norm[i];
    if (d->rope_half_dim) {
        if (!d->rope_cos || !d->rope_sin) return QORA_HIP_E_INVALID;
        for (uint64_t i = 0; i < d->rope_positions * d->rope_half_dim; ++i) sum += (uint64_t)(d->rope_cos[i] + d->rope_sin[i]);
    }
    (void)sum;
    c->model = true;
    c->model_layers = d->num_layers;
    return QORA_HIP_OK;
}

namespace {

int failures = 0;

void check(bool ok, const std::string& what) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
        ++failures;
    }
}

struct HostModel {
    qora_host_model m{};
    std::vector<std::vector<uint8_t>> packed;
    std::vector<std::vector<uint16_t>> words;   // F16 data or Q4 scales
    std::vector<const void*> wd;
    std::vector<const uint16_t*> ws;
    std::vector<std::vector<uint16_t>> norms;
    std::vector<const uint16_t*> in, post;
    std::vector<uint8_t> emb_p;
    std::vector<uint16_t> emb_w, fin;
    std::vector<float> cos_t, sin_t;
    std::vector<uint8_t> flags;
};

void make_model(HostModel& h, uint32_t fmt) {
    qora_host_model& m = h.m;
    m.num_layers = 2; m.vocab = 64; m.hidden = 64; m.intermediate = 96;
    m.num_heads = 2; m.num_kv_heads = 1; m.head_dim = 32; m.num_kv_groups = 2; m.rope_half_dim = 16;
    m.format = fmt;
    const uint64_t H = 64, I = 96, qd = 64, kvd = 32;
    const uint64_t shapes[7][2] = {{H, qd}, {H, kvd}, {H, kvd}, {qd, H}, {H, I}, {H, I}, {I, H}};
    for (uint32_t l = 0; l < m.num_layers; ++l)
        for (int j = 0; j < 7; ++j) {
            const uint64_t k = shapes[j][0], n = shapes[j][1];
            if (fmt == 1) {
                h.packed.emplace_back(k * n / 2);
                h.words.emplace_back(k * n / 32);
                qora_synth_q4(5, 16 * l + j, k, n, h.packed.back().data(), h.words.back().data());
            } else {
                h.packed.emplace_back();
                h.words.emplace_back(k * n);
                qora_synth_f16(5, 16 * l + j, k * n, 0.02f, h.words.back().data());
            }
        }
    for (size_t i = 0; i < h.words.size(); ++i) {
        h.wd.push_back(fmt == 1 ? (const void*)h.packed[i].data() : (const void*)h.words[i].data());
        h.ws.push_back(fmt == 1 ? h.words[i].data() : nullptr);
    }
    for (uint32_t l = 0; l < 2 * m.num_layers + 1; ++l) {
        h.norms.emplace_back(H);
        qora_synth_f16(6, l, H, 0.5f, h.norms.back().data());
    }
    for (uint32_t l = 0; l < m.num_layers; ++l) {
        h.in.push_back(h.norms[2 * l].data());
        h.post.push_back(h.norms[2 * l + 1].data());
    }
    if (fmt == 1) {
        h.emb_p.resize(m.vocab * H / 2);
        h.emb_w.resize(m.vocab * H / 32);
        qora_synth_q4(5, 1000, m.vocab, H, h.emb_p.data(), h.emb_w.data());
    } else {
        h.emb_w.resize(m.vocab * H);
        qora_synth_f16(5, 1000, m.vocab * H, 0.02f, h.emb_w.data());
    }
    const uint64_t positions = 16;
    h.cos_t.resize(positions * m.rope_half_dim);
    h.sin_t.resize(positions * m.rope_half_dim);
    qora_rope_tables(positions, m.rope_half_dim, 5e6, h.cos_t.data(), h.sin_t.data());
    h.flags = {0, 1};
    m.w_data = h.wd.data();
    m.w_scales = fmt == 1 ? h.ws.data() : nullptr;
    m.input_norm = h.in.data();
    m.post_attn_norm = h.post.data();
    m.embed_data = fmt == 1 ? (const void*)h.emb_p.data() : (const void*)h.emb_w.data();
    m.embed_scales = fmt == 1 ? h.emb_w.data() : nullptr;
    m.final_norm = h.norms.back().data();
    m.rope_cos = h.cos_t.data();
    m.rope_sin = h.sin_t.data();
    m.rope_positions = positions;
    m.use_rope = h.flags.data();
}

std::vector<uint8_t> read_file(const std::string& p) {
    std::vector<uint8_t> b;
    FILE* f = std::fopen(p.c_str(), "rb");
    if (!f) return b;
    uint8_t buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
    std::fclose(f);
    return b;
}

void write_file(const std::string& p, const std::vector<uint8_t>& b, size_t len) {
    FILE* f = std::fopen(p.c_str(), "wb");
    if (!f) { check(false, "cannot write " + p); return; }
    if (len) std::fwrite(b.data(), 1, len, f);
    std::fclose(f);
}

size_t alive(const qora_hip_ctx& c) {
    size_t n = 0;
    for (const Upload& u : c.w) n += u.alive;
    return n;
}

// One load of `b` (first `len` bytes); returns the status. A refused load
// must leave no upload alive.
int load(const std::string& path, const std::vector<uint8_t>& b, size_t len, const std::string& what) {
    write_file(path, b, len);
    qora_hip_ctx c;
    const int rc = qora_hip_load_model(&c, path.c_str(), 0, 0);
    if (rc != QORA_HIP_OK) check(alive(c) == 0 && !c.model, what + ": a refused load left uploads alive");
    else check(c.model, what + ": loaded without a model");
    return rc;
}

// xorshift64 for the corruption positions
uint64_t rng_state = 0x2545F4914F6CDD1Dull;
uint64_t next_u64() {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return rng_state;
}

void run_format(const std::string& dir, uint32_t fmt) {
    const std::string tag = fmt == 1 ? "q4" : "f16";
    HostModel h;
    make_model(h, fmt);
    const std::string path = dir + "/model_" + tag + ".qora";
    check(qora_file_write(path.c_str(), &h.m) == QORA_HIP_OK, tag + ": write");
    const std::vector<uint8_t> good = read_file(path);
    check(good.size() > 1000, tag + ": file size");

    // 1. round trip
    {
        qora_hip_ctx c;
        check(qora_hip_load_model(&c, path.c_str(), 0, 0) == QORA_HIP_OK, tag + ": valid file refused");
        check(c.model && c.model_layers == 2, tag + ": model");
        check(c.w.size() == 15, tag + ": upload count");
        for (size_t i = 0; i < 14 && i < c.w.size(); ++i) {
            if (fmt == 1) {
                check(c.w[i].a == h.packed[i] && c.w[i].b == h.words[i], tag + ": weight bytes " + std::to_string(i));
            } else {
                check(c.w[i].b == h.words[i], tag + ": weight words " + std::to_string(i));
            }
        }
    }
    // 2. truncations
    const size_t n = good.size();
    for (size_t len = 0; len < n; len += (len < 512 ? 1 : 97))
        check(load(path + ".t", good, len, tag + ": truncated at " + std::to_string(len)) != QORA_HIP_OK,
              tag + ": truncated file at " + std::to_string(len) + " loaded");
    // 3a. random byte and bit corruptions
    for (int it = 0; it < 1500; ++it) {
        std::vector<uint8_t> b = good;
        const int flips = 1 + (int)(next_u64() % 4);
        for (int f = 0; f < flips; ++f) {
            const size_t at = (size_t)(next_u64() % (it % 2 ? 600 : n));   // half of them in the header region
            if (next_u64() & 1) b[at] ^= (uint8_t)(1u << (next_u64() % 8));
            else b[at] = (uint8_t)next_u64();
        }
        (void)load(path + ".c", b, b.size(), tag + ": corruption " + std::to_string(it));
    }
    // 3b. 8 bytes of 0xFF (a huge length or count) at every offset of the first 600 bytes
    for (size_t at = 0; at + 8 <= std::min<size_t>(n, 600); ++at) {
        std::vector<uint8_t> b = good;
        std::memset(&b[at], 0xFF, 8);
        (void)load(path + ".l", b, b.size(), tag + ": 0xFF run at " + std::to_string(at));
    }
    std::remove((path + ".t").c_str());
    std::remove((path + ".c").c_str());
    std::remove((path + ".l").c_str());
    std::remove(path.c_str());
}

}  // namespace

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : ".";
    run_format(dir, 1);
    run_format(dir, 0);
    // the generator over odd sizes and both thread paths
    std::vector<uint8_t> p(97 * 64 / 2);
    std::vector<uint16_t> s(97 * 64 / 32), f(4099);
    std::vector<float> x(4099);
    std::vector<uint32_t> t(333);
    qora_synth_q4(1, 2, 97, 64, p.data(), s.data());
    qora_synth_f16(1, 3, f.size(), 0.02f, f.data());
    qora_synth_f32(1, 4, x.size(), x.data());
    qora_synth_tokens(1, 5, t.size(), 1000, t.data());
    for (uint32_t v : t) check(v < 1000, "token range");
    std::vector<uint8_t> big(2048 * 4096 / 2);
    std::vector<uint16_t> bigs(2048 * 4096 / 32);
    qora_synth_q4(1, 6, 2048, 4096, big.data(), bigs.data());
    if (failures) {
        std::fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    std::printf("qora_file_fuzz: all cases held\n");
    return 0;
}
