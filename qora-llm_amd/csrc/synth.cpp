// Seeded synthetic inputs in the reference's weight layout (host only).
//
// Every value is a pure function of (seed, tensor id, element index):
//   key  = mix64(seed ^ mix64(tensor_id + C))
//   r_i  = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)   (splitmix64 output i)
// so tensors can be generated in parallel, in any order, bit for bit.
// Normals are Box-Muller draws: u1, u2 = the high and low 32 bits of r_i
// (+ 1/2, times 2^-32), z = sqrt(-2 ln u1) cos(2 pi (u2 - 1/2)) (tails to
// 6.8 sigma). ln and cos are evaluated here from + - * / and sqrt alone
// (frexp, an atanh series for ln, a halved-angle Taylor series for cos), all
// correctly rounded in float64, so the numpy restatement used by the tests
// reproduces every byte.
#include "../../include/qora_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t tensor_id) {
    return mix64(seed ^ mix64(tensor_id + 0x632BE59BD9B4E019ull));
}

inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

// ln u for 0 < u <= 1: u = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m =
// 2 atanh(t) = 2 t sum_k t^(2k) / (2k + 1), t = (m - 1) / (m + 1), |t| < 0.172
// (terms to t^22).
inline double ln_unit(double u) {
    int e = 0;
    double m = std::frexp(u, &e);                  // u = m 2^e, m in [1/2, 1)
    if (m < 0.70710678118654752) {
        m = m * 2.0;
        e = e - 1;
    }
    const double t = (m - 1.0) / (m + 1.0), t2 = t * t;
    double s = 1.0 / 23.0;
    for (int k = 10; k >= 0; --k) s = s * t2 + 1.0 / (2.0 * k + 1.0);
    return (double)e * 0.6931471805599453 + 2.0 * t * s;
}

// (-1)^k / (2k)!, k = 0..12, by repeated division
struct CosCoef {
    double c[13];
    CosCoef() {
        c[0] = 1.0;
        for (int k = 1; k <= 12; ++k) c[k] = -c[k - 1] / ((2.0 * k - 1.0) * (2.0 * k));
    }
};
const CosCoef kCos;

// cos x for |x| <= pi: cos x = 2 cos^2(x / 2) - 1, cos(x / 2) by its Taylor
// series to (x / 2)^24.
inline double cos_pm_pi(double x) {
    const double h = 0.5 * x, h2 = h * h;
    double c = kCos.c[12];
    for (int k = 11; k >= 0; --k) c = c * h2 + kCos.c[k];
    return 2.0 * c * c - 1.0;
}

inline double normal_of(uint64_t r) {
    const double u1 = ((double)(r >> 32) + 0.5) * 2.3283064365386963e-10;          // 2^-32
    const double u2 = ((double)(r & 0xFFFFFFFFull) + 0.5) * 2.3283064365386963e-10;
    return std::sqrt(-2.0 * ln_unit(u1)) * cos_pm_pi(6.283185307179586 * (u2 - 0.5));
}

// binary32 -> binary16, round to nearest even.
uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0u));
    if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (absx < 0x38800000u) {
        if (absx < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = absx >> 23;
        const uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        const uint32_t sh = 126 - e;
        uint32_t r = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u);
        const uint32_t half = 1u << (sh - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (absx >> 13) - (112u << 10);
    const uint32_t rem = absx & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

// Run fn(begin, end) over [0, count) on the host cores.
template <class F>
void parallel_for(uint64_t count, F fn) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    nt = std::min<unsigned>(nt, 32);
    if (count < (1u << 20) || nt == 1) {
        fn(0, count);
        return;
    }
    std::vector<std::thread> ts;
    const uint64_t chunk = (count + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const uint64_t b = (uint64_t)t * chunk, e = std::min<uint64_t>(count, b + chunk);
        if (b >= e) break;
        ts.emplace_back([=] { fn(b, e); });
    }
    for (auto& th : ts) th.join();
}

}  // namespace

extern "C" void qora_synth_q4(uint64_t seed, uint64_t tensor_id, uint64_t k, uint64_t n, uint8_t* packed,
                              uint16_t* scales) {
    const uint64_t nbytes = k * n / 2;
    const uint64_t key_q = stream_key(seed, tensor_id * 2);
    const uint64_t key_s = stream_key(seed, tensor_id * 2 + 1);
    // one 64-bit draw per 4 bytes (8 nibbles, 8 bits each); v = U{0..14}
    parallel_for((nbytes + 3) / 4, [&](uint64_t b, uint64_t e) {
        for (uint64_t j = b; j < e; ++j) {
            const uint64_t r = draw(key_q, j);
            for (int m = 0; m < 4; ++m) {
                const uint64_t idx = j * 4 + (uint64_t)m;
                if (idx >= nbytes) break;
                const uint32_t u_lo = (uint32_t)(r >> (16 * m)) & 0xFFu;
                const uint32_t u_hi = (uint32_t)(r >> (16 * m + 8)) & 0xFFu;
                const uint32_t q_lo = ((u_lo * 15u) >> 8) + 1u;   // v + 8, v in [-7, 7]
                const uint32_t q_hi = ((u_hi * 15u) >> 8) + 1u;
                packed[idx] = (uint8_t)(q_lo | (q_hi << 4));
            }
        }
    });
    const uint64_t nscales = k * n / 32;
    const double mul = 0.02 / 7.0;
    parallel_for(nscales, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i)
            scales[i] = f2h((float)(std::fabs(normal_of(draw(key_s, i))) * mul));
    });
}

extern "C" void qora_synth_f16(uint64_t seed, uint64_t tensor_id, uint64_t count, float stddev, uint16_t* out) {
    const uint64_t key = stream_key(seed, tensor_id * 2);
    const double sd = (double)stddev;
    parallel_for(count, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i) out[i] = f2h((float)(normal_of(draw(key, i)) * sd));
    });
}

extern "C" void qora_synth_f32(uint64_t seed, uint64_t tensor_id, uint64_t count, float* out) {
    const uint64_t key = stream_key(seed, tensor_id * 2);
    parallel_for(count, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i) out[i] = (float)normal_of(draw(key, i));
    });
}

extern "C" void qora_synth_tokens(uint64_t seed, uint64_t tensor_id, uint64_t count, uint32_t vocab, uint32_t* out) {
    const uint64_t key = stream_key(seed, tensor_id * 2);
    for (uint64_t i = 0; i < count; ++i) out[i] = (uint32_t)(((draw(key, i) >> 32) * (uint64_t)vocab) >> 32);
}

extern "C" void qora_rope_tables(uint64_t positions, uint32_t half_dim, double theta, float* cos_out,
                                 float* sin_out) {
    std::vector<double> inv(half_dim);
    for (uint32_t i = 0; i < half_dim; ++i) inv[i] = std::pow(theta, -(2.0 * i) / (2.0 * half_dim));
    parallel_for(positions, [&](uint64_t b, uint64_t e) {
        for (uint64_t p = b; p < e; ++p)
            for (uint32_t i = 0; i < half_dim; ++i) {
                const double a = (double)p * inv[i];
                cos_out[p * half_dim + i] = (float)std::cos(a);
                sin_out[p * half_dim + i] = (float)std::sin(a);
            }
    });
}
