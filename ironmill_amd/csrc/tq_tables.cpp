// tq_tables.cpp -- TurboQuant table generation and upload (host side).
//
// Counterpart of MetalTurboQuantModel::new (metal/turboquant/mod.rs:221-287):
//  * rotation signs from a seeded generator (turboquant/rotation.rs:13-25),
//  * K codebook: Lloyd-Max for N(0, 1/sqrt(d)) with n_bits-1 bits, V codebook with
//    n_bits bits (turboquant/codebook.rs:20-52),
//  * QJL matrix S ~ N(0,1), seed + 1 (rotation.rs:31-49).
// The generator is ChaCha12 keyed by a PCG32 expansion of the u64 seed, the
// construction of rand's StdRng::seed_from_u64.  The Lloyd-Max iteration keeps
// the reference's starting quantiles and erf approximation because the 7/8-bit
// tables are still moving when the 200-iteration cap stops them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "imh_internal.h"

namespace {

double erf_as(double x) {  // Abramowitz & Stegun 7.1.26
    const double a1 = 0.254829592, a2 = -0.284496736, a3 = 1.421413741;
    const double a4 = -1.453152027, a5 = 1.061405429, p = 0.3275911;
    const double sign = x < 0.0 ? -1.0 : 1.0;
    const double ax = std::fabs(x);
    const double t = 1.0 / (1.0 + p * ax);
    const double y = 1.0 - (((((a5 * t + a4) * t) + a3) * t + a2) * t + a1) * t * std::exp(-ax * ax);
    return sign * y;
}

double gauss_cdf(double x) { return 0.5 * (1.0 + erf_as(x * 0.70710678118654752440)); }
double gauss_pdf(double x) { return std::exp(-0.5 * x * x) / std::sqrt(2.0 * 3.14159265358979323846); }

// Starting quantiles: rational approximations in the central and tail regions.
double start_quantile(double p) {
    if (p <= 0.0) return -INFINITY;
    if (p >= 1.0) return INFINITY;
    const double t = p - 0.5;
    if (std::fabs(t) <= 0.42) {
        const double r = t * t;
        const double num =
            t * (((2.5066282746310002 * r + 18.6150006252966) * r + 41.39119773534996) * r + 25.44106049637689);
        const double den = (((14.382029373388 * r + 63.690613) * r + 84.681) * r + 40.304) * r + 1.0;
        return num / den;
    }
    const double r = t < 0.0 ? p : 1.0 - p;
    const double s = std::sqrt(-std::log(r));
    double v;
    if (s <= 5.0) {
        const double u = s - 1.6;
        const double num =
            ((((((0.000124818987 * u + 0.0227061845) * u + 0.2728688) * u + 1.3058437) * u + 2.7580128) * u +
              2.2311569) * u + 0.6462025) * u + 0.001612;
        const double den =
            ((((((0.000038746 * u + 0.00745102) * u + 0.09234118) * u + 0.4710441) * u + 1.0507501) * u + 1.0) * u +
             0.2127601) * u + 1.0;
        v = num / den;
    } else {
        const double u = s - 5.0;
        v = (((((((0.0000000271 * u + 0.00000342556) * u + 0.000170717) * u + 0.004531901) * u + 0.06871337) * u +
               0.56419917) * u + 1.9715909) * u + 2.1538256) /
            (((((((0.0000000393 * u + 0.00000489649) * u + 0.000230147) * u + 0.005492439) * u + 0.06353648) * u +
               0.3445453) * u + 0.73741429) * u + 1.0);
    }
    return t < 0.0 ? -v : v;
}

double bin_mean(double sigma, double lo, double hi) {
    const double a = lo / sigma, b = hi / sigma;
    const double prob = gauss_cdf(b) - gauss_cdf(a);
    if (prob < 1e-30) {
        if (std::isinf(lo)) return hi;
        if (std::isinf(hi)) return lo;
        return (lo + hi) / 2.0;
    }
    return sigma * (gauss_pdf(a) - gauss_pdf(b)) / prob;
}

void lloyd_max(int dim, int bits, std::vector<float> &levels, std::vector<float> &bounds) {
    const int n = 1 << bits;
    const double sigma = 1.0 / std::sqrt((double)dim);
    std::vector<double> lv(n), nl(n), bd(n > 1 ? n - 1 : 1);
    for (int i = 0; i < n; i++) lv[i] = sigma * start_quantile(((double)i + 0.5) / (double)n);
    for (int it = 0; it < 200; it++) {
        for (int i = 0; i + 1 < n; i++) bd[i] = (lv[i] + lv[i + 1]) / 2.0;
        for (int i = 0; i < n; i++)
            nl[i] = bin_mean(sigma, i == 0 ? -INFINITY : bd[i - 1], i == n - 1 ? INFINITY : bd[i]);
        double delta = 0.0;
        for (int i = 0; i < n; i++) {
            delta = std::fmax(delta, std::fabs(lv[i] - nl[i]));
            lv[i] = nl[i];
        }
        if (delta < 1e-10) break;
    }
    levels.resize(n);
    bounds.resize(n - 1);
    for (int i = 0; i + 1 < n; i++) bounds[i] = (float)((lv[i] + lv[i + 1]) / 2.0);
    for (int i = 0; i < n; i++) levels[i] = (float)lv[i];
}

// ChaCha12 keyed from a u64 seed, read 64 bits at a time.
class SeededStream {
  public:
    explicit SeededStream(uint64_t seed) {
        uint64_t st = seed;
        for (int i = 0; i < 8; i++) {
            st = st * 6364136223846793005ULL + 11634580027462260723ULL;
            const uint32_t xs = (uint32_t)(((st >> 18) ^ st) >> 27);
            const uint32_t rot = (uint32_t)(st >> 59);
            key_[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
        }
    }
    uint64_t next_u64() {
        if (pos_ >= 64) refill();
        const uint64_t lo = buf_[pos_], hi = buf_[pos_ + 1];
        pos_ += 2;
        return (hi << 32) | lo;
    }
    double next_unit() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }

  private:
    static uint32_t rotl(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }
    static void quarter(uint32_t &a, uint32_t &b, uint32_t &c, uint32_t &d) {
        a += b; d ^= a; d = rotl(d, 16);
        c += d; b ^= c; b = rotl(b, 12);
        a += b; d ^= a; d = rotl(d, 8);
        c += d; b ^= c; b = rotl(b, 7);
    }
    void refill() {
        for (int blk = 0; blk < 4; blk++) {
            uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
            for (int i = 0; i < 8; i++) in[4 + i] = key_[i];
            const uint64_t c = ctr_ + (uint64_t)blk;
            in[12] = (uint32_t)c;
            in[13] = (uint32_t)(c >> 32);
            in[14] = 0;
            in[15] = 0;
            uint32_t x[16];
            std::memcpy(x, in, sizeof(x));
            for (int r = 0; r < 12; r += 2) {
                quarter(x[0], x[4], x[8], x[12]);
                quarter(x[1], x[5], x[9], x[13]);
                quarter(x[2], x[6], x[10], x[14]);
                quarter(x[3], x[7], x[11], x[15]);
                quarter(x[0], x[5], x[10], x[15]);
                quarter(x[1], x[6], x[11], x[12]);
                quarter(x[2], x[7], x[8], x[13]);
                quarter(x[3], x[4], x[9], x[14]);
            }
            for (int i = 0; i < 16; i++) buf_[16 * blk + i] = x[i] + in[i];
        }
        ctr_ += 4;
        pos_ = 0;
    }
    uint32_t key_[8];
    uint32_t buf_[64];
    uint64_t ctr_ = 0;
    int pos_ = 64;
};

int upload(imh_device *dev, uint32_t d, uint32_t bits, const float *signs, const float *kcb,
           const float *kbd, const float *vcb, const float *vbd, const float *qjl,
           imh_tq_tables **out) {
    const size_t nk = (size_t)1 << (bits - 1), nv = (size_t)1 << bits;
    const size_t dd = (size_t)d * d;
    const size_t total = d + nk + (nk - 1) + nv + (nv - 1) + 2 * dd;
    std::vector<float> host(total);
    size_t o = 0;
    auto put = [&](const float *src, size_t n) {
        std::memcpy(host.data() + o, src, n * sizeof(float));
        o += n;
    };
    put(signs, d);
    put(kcb, nk);
    put(kbd, nk - 1);
    put(vcb, nv);
    put(vbd, nv - 1);
    put(qjl, dd);
    for (size_t k = 0; k < d; k++)
        for (size_t i = 0; i < d; i++) host[o + k * d + i] = qjl[i * d + k];  // transposed copy
    o += dd;
    int rc = imh::use_device(dev);
    if (rc) return rc;
    float *base = nullptr;
    IMH_HIP(hipMalloc(&base, total * sizeof(float)));
    hipError_t e = hipMemcpy(base, host.data(), total * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return imh::hip_fail(e, "hipMemcpy(tq tables)");
    }
    imh_tq_tables *t = new (std::nothrow) imh_tq_tables();
    if (!t) {
        (void)hipFree(base);
        return imh::fail(IMH_ENOMEM, "imh_tq_tables: host allocation failed");
    }
    t->dev = dev;
    t->head_dim = d;
    t->n_bits = bits;
    t->base = base;
    t->total_floats = total;
    t->signs = base;
    t->k_codebook = t->signs + d;
    t->k_bounds = t->k_codebook + nk;
    t->v_codebook = t->k_bounds + (nk - 1);
    t->v_bounds = t->v_codebook + nv;
    t->qjl = t->v_bounds + (nv - 1);
    t->qjl_t = t->qjl + dd;
    // search tables for the index rule (see imh_tq_tables)
    auto build = [](const float *bd, size_t n, std::vector<float> &sv, std::vector<int32_t> &pm) {
        std::vector<std::pair<float, int32_t>> e;
        for (size_t j = 0; j < n; j++)
            if (!std::isnan(bd[j])) e.emplace_back(bd[j], (int32_t)(j + 1));
        std::stable_sort(e.begin(), e.end(), [](const auto &x, const auto &y) { return x.first < y.first; });
        int32_t run = 0;
        for (const auto &p : e) {
            run = std::max(run, p.second);
            sv.push_back(p.first);
            pm.push_back(run);
        }
    };
    std::vector<float> ks, vs;
    std::vector<int32_t> kp, vp;
    build(kbd, nk - 1, ks, kp);
    build(vbd, nv - 1, vs, vp);
    const size_t sbytes = 4 * (2 * ks.size() + 2 * vs.size()) + 16;
    std::vector<uint8_t> sh(sbytes, 0);
    size_t so = 0;
    auto put_bytes = [&](const void *src, size_t bytes) {
        std::memcpy(sh.data() + so, src, bytes);
        so += bytes;
    };
    put_bytes(ks.data(), 4 * ks.size());
    put_bytes(kp.data(), 4 * kp.size());
    put_bytes(vs.data(), 4 * vs.size());
    put_bytes(vp.data(), 4 * vp.size());
    e = hipMalloc(&t->search_base, sbytes);
    if (e == hipSuccess) e = hipMemcpy(t->search_base, sh.data(), sbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (t->search_base) (void)hipFree(t->search_base);
        (void)hipFree(base);
        delete t;
        return imh::hip_fail(e, "imh_tq_tables: search tables");
    }
    uint8_t *sb = static_cast<uint8_t *>(t->search_base);
    t->k_search = (int)ks.size();
    t->v_search = (int)vs.size();
    t->k_sorted = reinterpret_cast<const float *>(sb);
    t->k_prefmax = reinterpret_cast<const int32_t *>(sb + 4 * ks.size());
    t->v_sorted = reinterpret_cast<const float *>(sb + 8 * ks.size());
    t->v_prefmax = reinterpret_cast<const int32_t *>(sb + 8 * ks.size() + 4 * vs.size());
    *out = t;
    return IMH_OK;
}

int check_shape(const char *who, uint32_t d, uint32_t bits) {
    if (d == 0 || (d & (d - 1)) != 0)
        return imh::fail(IMH_EINVAL, std::string(who) + ": head_dim " + std::to_string(d) +
                                         " must be a power of two for the Walsh-Hadamard butterfly");
    if (bits < 2 || bits > 8)
        return imh::fail(IMH_EINVAL, std::string(who) + ": n_bits must be in [2, 8]");
    if (d != 128 || bits != 8)
        return imh::fail(IMH_EUNSUPPORTED, std::string(who) + ": kernels are built for head_dim 128, n_bits 8");
    return IMH_OK;
}

}  // namespace

extern "C" {

int imh_tq_tables_create(imh_device *dev, uint32_t head_dim, uint32_t n_bits, uint64_t rotation_seed,
                         imh_tq_tables **out) {
    const char *who = "imh_tq_tables_create";
    if (!dev || !out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    *out = nullptr;
    int rc = check_shape(who, head_dim, n_bits);
    if (rc) return rc;
    std::vector<float> signs(head_dim), qjl((size_t)head_dim * head_dim);
    {
        SeededStream rng(rotation_seed);
        for (uint32_t i = 0; i < head_dim; i++) signs[i] = rng.next_u64() < (1ULL << 63) ? 1.0f : -1.0f;
    }
    {
        SeededStream rng(rotation_seed + 1);
        const double two_pi = 2.0 * 3.14159265358979323846;
        size_t i = 0, n = qjl.size();
        while (i < n) {
            double u1 = rng.next_unit();
            const double u2 = rng.next_unit();
            if (u1 < 1e-300) u1 = 1e-300;
            const double r = std::sqrt(-2.0 * std::log(u1));
            qjl[i++] = (float)(r * std::cos(two_pi * u2));
            if (i < n) qjl[i++] = (float)(r * std::sin(two_pi * u2));
        }
    }
    std::vector<float> kcb, kbd, vcb, vbd;
    lloyd_max((int)head_dim, (int)n_bits - 1, kcb, kbd);
    lloyd_max((int)head_dim, (int)n_bits, vcb, vbd);
    return upload(dev, head_dim, n_bits, signs.data(), kcb.data(), kbd.data(), vcb.data(), vbd.data(),
                  qjl.data(), out);
}

int imh_tq_tables_create_from_host(imh_device *dev, uint32_t head_dim, uint32_t n_bits, const float *signs,
                                   const float *k_codebook, const float *k_bounds, const float *v_codebook,
                                   const float *v_bounds, const float *qjl, imh_tq_tables **out) {
    const char *who = "imh_tq_tables_create_from_host";
    if (!dev || !out || !signs || !k_codebook || !k_bounds || !v_codebook || !v_bounds || !qjl)
        return imh::fail(IMH_EINVAL, std::string(who) + ": NULL argument");
    *out = nullptr;
    int rc = check_shape(who, head_dim, n_bits);
    if (rc) return rc;
    return upload(dev, head_dim, n_bits, signs, k_codebook, k_bounds, v_codebook, v_bounds, qjl, out);
}

void imh_tq_tables_free(imh_tq_tables *t) {
    if (!t) return;
    imh::use_device(t->dev);
    (void)hipFree(t->base);
    if (t->search_base) (void)hipFree(t->search_base);
    delete t;
}

int imh_tq_tables_read(const imh_tq_tables *t, int which, float *dst, size_t capacity, size_t *count) {
    if (!t || !count) return imh::fail(IMH_EINVAL, "imh_tq_tables_read: NULL argument");
    const size_t nk = (size_t)1 << (t->n_bits - 1), nv = (size_t)1 << t->n_bits;
    const float *src;
    size_t n;
    switch (which) {
        case IMH_TQ_SIGNS: src = t->signs; n = t->head_dim; break;
        case IMH_TQ_K_CODEBOOK: src = t->k_codebook; n = nk; break;
        case IMH_TQ_K_BOUNDS: src = t->k_bounds; n = nk - 1; break;
        case IMH_TQ_V_CODEBOOK: src = t->v_codebook; n = nv; break;
        case IMH_TQ_V_BOUNDS: src = t->v_bounds; n = nv - 1; break;
        case IMH_TQ_QJL: src = t->qjl; n = (size_t)t->head_dim * t->head_dim; break;
        default: return imh::fail(IMH_EINVAL, "imh_tq_tables_read: unknown table id");
    }
    *count = n;
    if (!dst) return IMH_OK;
    if (capacity < n) return imh::fail(IMH_EINVAL, "imh_tq_tables_read: destination too small");
    int rc = imh::use_device(t->dev);
    if (rc) return rc;
    IMH_HIP(hipMemcpy(dst, src, n * sizeof(float), hipMemcpyDeviceToHost));
    return IMH_OK;
}

int imh_tq_cache_sizes(uint32_t batch, uint32_t num_kv_heads, uint32_t head_dim, uint32_t max_seq_len,
                       size_t *codes_bytes, size_t *scale_bytes) {
    if (!codes_bytes || !scale_bytes) return imh::fail(IMH_EINVAL, "imh_tq_cache_sizes: NULL argument");
    const unsigned __int128 pos = (unsigned __int128)batch * num_kv_heads * max_seq_len;
    const unsigned __int128 codes = pos * head_dim;
    if (codes > (unsigned __int128)SIZE_MAX / 4)
        return imh::fail(IMH_EINVAL, "imh_tq_cache_sizes: cache size overflows size_t");
    *codes_bytes = (size_t)codes;
    *scale_bytes = (size_t)pos * sizeof(float);
    return IMH_OK;
}

}  // extern "C"
