// Host implementations of the ops (see cpu_kernels.hpp). The formulas are the
// reference README's (README.md:157-292) and its op tests' torch statements
// (test/ops/*.py), the same ones the HIP kernels follow.
#include "cpu_kernels.hpp"

#include "../../common.hpp"

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <mutex>
#include <sched.h>
#include <cmath>
#include <cstdlib>
#include <limits>
#include <thread>
#include <type_traits>
#include <vector>

namespace llaisys::cpu {

namespace {

using kernels::kHeadDim;
using kernels::kPageElems;
using kernels::kPageTokens;

constexpr int kErrBadBlock = 1;
constexpr int kErrTooLong = 2;
constexpr int kErrBadIndex = 4;

void raiseFlag(int *err, int bit) { __atomic_fetch_or(err, bit, __ATOMIC_RELAXED); }

// f32 -> IEEE binary16, round to nearest even; overflow to inf, NaN kept quiet.
uint16_t f32ToF16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t abs = u & 0x7fffffffu;
    if (abs > 0x7f800000u) return uint16_t(sign | 0x7e00u);
    if (abs >= 0x477ff000u) return uint16_t(sign | 0x7c00u); // rounds to >= 65520: inf
    if (abs < 0x38800000u) {                                 // below 2^-14: subnormal half
        // value = abs_f * 2^24 half-ulps; round the 24+ bit mantissa by hand.
        if (abs < 0x33000000u) return uint16_t(sign); // below 2^-25: rounds to zero
        const uint32_t e = abs >> 23;
        const uint32_t m = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e; // m * 2^(e-150) in units of 2^-24: m >> (150-e-24)
        const uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        const uint32_t r = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
        return uint16_t(sign | r);
    }
    // normal: rebias exponent (127 -> 15) and round 23 -> 10 mantissa bits
    uint32_t h = ((abs - 0x38000000u) >> 13);
    const uint32_t rem = abs & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return uint16_t(sign | h);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
    static float ld(const void *p, size_t i) { return static_cast<const float *>(p)[i]; }
    static void st(void *p, size_t i, float v) { static_cast<float *>(p)[i] = v; }
};
struct F16 {};
struct BF16 {};
template <> struct Elem<F16> {
    static float ld(const void *p, size_t i) { return f16ToF32(static_cast<const uint16_t *>(p)[i]); }
    static void st(void *p, size_t i, float v) { static_cast<uint16_t *>(p)[i] = f32ToF16(v); }
};
template <> struct Elem<BF16> {
    static float ld(const void *p, size_t i) { return bf16ToF32(static_cast<const uint16_t *>(p)[i]); }
    static void st(void *p, size_t i, float v) { static_cast<uint16_t *>(p)[i] = f32ToBf16(v); }
};

template <template <typename> class F, typename... Args> void byType(ElemType t, Args &&...args) {
    switch (t) {
    case ElemType::F32: return F<float>::run(args...);
    case ElemType::F16: return F<F16>::run(args...);
    case ElemType::BF16: return F<BF16>::run(args...);
    }
}

float ldAny(ElemType t, const void *p, size_t i) {
    switch (t) {
    case ElemType::F32: return Elem<float>::ld(p, i);
    case ElemType::F16: return Elem<F16>::ld(p, i);
    default: return Elem<BF16>::ld(p, i);
    }
}

// Widen n elements of any float type to fp32.
void widen(float *dst, const void *src, ElemType t, size_t n);

// A persistent pool of threads() - 1 workers. One job runs at a time: a job
// is a range [0, n) handed out in chunks through an atomic cursor; the caller
// works on it too and returns when every chunk is done. A parallelFor issued
// while another is running (another host thread, or nested) runs inline.
class Pool {
public:
    static Pool &get() {
        // Destroyed at exit (its workers joined); no job runs past main's return.
        static Pool pool(threads() - 1);
        static Pool *p = &pool;
        return *p;
    }

    template <typename Fn> void run(size_t n, size_t chunk, Fn &fn) {
        std::unique_lock<std::mutex> busy(busy_, std::try_to_lock);
        if (!busy.owns_lock() || workers_.empty()) {
            for (size_t i = 0; i < n; ++i) fn(i);
            return;
        }
        auto body = [](void *ctx, size_t i) { (*static_cast<Fn *>(ctx))(i); };
        {
            std::lock_guard<std::mutex> g(m_);
            job_ = {body, &fn, n, chunk};
            cursor_.store(0);
            pending_ = workers_.size();
            ++generation_;
        }
        cv_.notify_all();
        work(job_);
        std::unique_lock<std::mutex> g(m_);
        done_.wait(g, [&] { return pending_ == 0; });
    }

private:
    struct Job {
        void (*body)(void *, size_t);
        void *ctx;
        size_t n, chunk;
    };

    explicit Pool(int nworkers) {
        for (int i = 0; i < nworkers; ++i) workers_.emplace_back([this] { loop(); });
    }

    // At process exit the workers leave their wait and are joined, so no
    // thread outlives the library.
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &w : workers_)
            if (w.joinable()) w.join();
    }

    void work(const Job &j) {
        for (;;) {
            const size_t s = cursor_.fetch_add(j.chunk);
            if (s >= j.n) return;
            const size_t e = std::min(j.n, s + j.chunk);
            for (size_t i = s; i < e; ++i) j.body(j.ctx, i);
        }
    }

    void loop() {
        uint64_t seen = 0;
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [&] { return stop_ || generation_ != seen; });
                if (stop_) return;
                seen = generation_;
                j = job_;
            }
            work(j);
            std::lock_guard<std::mutex> g(m_);
            if (--pending_ == 0) done_.notify_one();
        }
    }

    std::vector<std::thread> workers_;
    std::mutex busy_, m_;
    std::condition_variable cv_, done_;
    Job job_{};
    std::atomic<size_t> cursor_{0};
    size_t pending_ = 0;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

// Run fn(i) for i in [0, n) over the host threads, in chunks of at least
// `grain` items (one thread when n <= grain).
template <typename Fn> void parallelFor(size_t n, size_t grain, Fn &&fn) {
    if (n == 0) return;
    grain = std::max<size_t>(grain, 1);
    if (n <= grain || threads() == 1) {
        for (size_t i = 0; i < n; ++i) fn(i);
        return;
    }
    const size_t chunk = std::max(grain, n / (size_t(threads()) * 8) + 1);
    Pool::get().run(n, chunk, fn);
}

void widen(float *dst, const void *src, ElemType t, size_t n) {
    if (t == ElemType::F32) {
        std::memcpy(dst, src, n * sizeof(float));
        return;
    }
    parallelFor(n, 1 << 16, [&](size_t i) { dst[i] = ldAny(t, src, i); });
}

inline int kIndex(int t, int d) { return (d >> 3) * 128 + t * 8 + (d & 7); }
inline int vIndex(int t, int d) { return (d >> 5) * 512 + (t >> 2) * 128 + (d & 15) * 8 + ((d >> 4) & 1) * 4 + (t & 3); }

// Largest b with cu[b] <= r.
int owningSequence(const int32_t *cu, int B, int r) {
    return int(std::upper_bound(cu, cu + B, r) - cu) - 1;
}

float dot(const float *a, const float *b, int n) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        s0 += a[i] * b[i];
        s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2];
        s3 += a[i + 3] * b[i + 3];
    }
    for (; i < n; ++i) s0 += a[i] * b[i];
    return (s0 + s1) + (s2 + s3);
}

// softmax(scale * q . K^T) V over `n` keys: scores into s[n] (fp32), result
// into o[dv] (fp32). Keys with skip[j] set are left out; all skipped -> zeros.
void attendRow(float *o, float *s, const float *q, const float *K, const float *V, int n, int d, int dv,
               size_t kstride, size_t vstride, float scale, const uint8_t *skip) {
    float m = -std::numeric_limits<float>::infinity();
    for (int j = 0; j < n; ++j) {
        s[j] = (skip && skip[j]) ? -std::numeric_limits<float>::infinity() : scale * dot(q, K + j * kstride, d);
        m = std::max(m, s[j]);
    }
    std::fill(o, o + dv, 0.f);
    if (!(m > -std::numeric_limits<float>::infinity())) return;
    float l = 0.f;
    for (int j = 0; j < n; ++j) {
        const float p = std::exp(s[j] - m);
        l += p;
        if (p == 0.f) continue;
        const float *vr = V + j * vstride;
        for (int c = 0; c < dv; ++c) o[c] += p * vr[c];
    }
    const float inv = 1.f / l;
    for (int c = 0; c < dv; ++c) o[c] *= inv;
}

template <typename T> struct AddOp {
    static void run(void *c, const void *a, const void *b, size_t n) {
        parallelFor(n, 1 << 15, [&](size_t i) { Elem<T>::st(c, i, Elem<T>::ld(a, i) + Elem<T>::ld(b, i)); });
    }
};

template <typename T> struct SwigluOp {
    static void run(void *o, const void *g, const void *u, size_t n) {
        parallelFor(n, 1 << 15, [&](size_t i) {
            const float gv = Elem<T>::ld(g, i);
            Elem<T>::st(o, i, Elem<T>::ld(u, i) * gv / (1.f + std::exp(-gv)));
        });
    }
};

template <typename T> struct RmsOp {
    static void run(void *o, const void *x, const void *w, size_t rows, int d, float eps) {
        parallelFor(rows, 16, [&](size_t r) {
            float ss = 0.f;
            for (int c = 0; c < d; ++c) {
                const float v = Elem<T>::ld(x, r * d + c);
                ss += v * v;
            }
            const float inv = 1.f / std::sqrt(ss / float(d) + eps);
            for (int c = 0; c < d; ++c) Elem<T>::st(o, r * d + c, Elem<T>::ld(x, r * d + c) * inv * Elem<T>::ld(w, c));
        });
    }
};

template <typename T> struct RopeOp {
    static void run(void *o, const void *x, const int64_t *pos, size_t ntok, int nhead, int d, float theta) {
        const int half = d / 2;
        parallelFor(ntok, 4, [&](size_t tok) {
            const float p = float(pos[tok]);
            for (int h = 0; h < nhead; ++h) {
                const size_t base = (tok * nhead + h) * size_t(d);
                for (int j = 0; j < half; ++j) {
                    const float phi = p / std::pow(theta, float(2 * j) / float(d));
                    const float s = std::sin(phi), c = std::cos(phi);
                    const float a = Elem<T>::ld(x, base + j), b = Elem<T>::ld(x, base + half + j);
                    Elem<T>::st(o, base + j, a * c - b * s);
                    Elem<T>::st(o, base + half + j, b * c + a * s);
                }
            }
        });
    }
};

// Order-preserving key of a value: a NaN ranks above +inf (torch.max
// propagates NaN) and +0 above -0, so the largest key is the maximum.
inline uint32_t orderKey(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if (v != v) u = 0x7fc00000u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <typename T> struct ArgmaxOp {
    static void run(int64_t *idx, void *val, const void *vals, size_t rows, int64_t n) {
        parallelFor(rows, 1, [&](size_t r) {
            // First column holding the largest key.
            int64_t best = 0;
            uint32_t bk = orderKey(Elem<T>::ld(vals, r * n));
            for (int64_t c = 1; c < n; ++c) {
                const uint32_t k = orderKey(Elem<T>::ld(vals, r * n + c));
                if (k > bk) {
                    bk = k;
                    best = c;
                }
            }
            idx[r] = best;
            if (val) {
                const size_t esz = std::is_same<T, float>::value ? 4 : 2;
                std::memcpy(static_cast<std::byte *>(val) + r * esz,
                            static_cast<const std::byte *>(vals) + (r * n + best) * esz, esz);
            }
        });
    }
};

} // namespace

int threads() {
    static const int n = [] {
        if (const char *e = std::getenv("LLAISYS_CPU_THREADS")) {
            const int v = std::atoi(e);
            if (v > 0) return v;
        }
        // the CPUs this process may run on (a container's share), not the machine's
        cpu_set_t set;
        if (sched_getaffinity(0, sizeof(set), &set) == 0 && CPU_COUNT(&set) > 0) return CPU_COUNT(&set);
        return int(std::max(1u, std::thread::hardware_concurrency()));
    }();
    return n;
}

void add(void *c, const void *a, const void *b, ElemType t, size_t n) { byType<AddOp>(t, c, a, b, n); }
void swiglu(void *out, const void *gate, const void *up, ElemType t, size_t n) { byType<SwigluOp>(t, out, gate, up, n); }
void rmsNorm(void *out, const void *x, const void *w, ElemType t, size_t rows, int d, float eps) {
    byType<RmsOp>(t, out, x, w, rows, d, eps);
}
void rope(void *out, const void *in, const int64_t *pos, ElemType t, size_t ntok, int nhead, int d, float theta) {
    byType<RopeOp>(t, out, in, pos, ntok, nhead, d, theta);
}
void argmax(int64_t *idx, void *val, const void *vals, ElemType t, size_t rows, int64_t n) {
    byType<ArgmaxOp>(t, idx, val, vals, rows, n);
}

void embedding(void *out, const int64_t *idx, const void *weight, ElemType t, size_t rows, int64_t vocab, int d,
               int *err) {
    const size_t esz = t == ElemType::F32 ? 4 : 2;
    parallelFor(rows, 64, [&](size_t r) {
        const int64_t i = idx[r];
        if (i < 0 || i >= vocab) {
            raiseFlag(err, kErrBadIndex);
            return;
        }
        std::memcpy(static_cast<std::byte *>(out) + r * d * esz, static_cast<const std::byte *>(weight) + size_t(i) * d * esz,
                    d * esz);
    });
}

// Tiles of 4 rows x 4 output columns per task keep 16 accumulators in
// registers and reuse each loaded X/W element 4 times. Elements are widened
// as they are read, so no fp32 copy of the weight is made (an LM head's
// would be ~1 GB).
template <typename T> struct LinearOp {
    static void run(void *out, const void *in, const void *weight, const void *bias, int M, int N, int K) {
        const int mt = (M + 3) / 4, nt = (N + 3) / 4;
        parallelFor(size_t(mt) * nt, 4, [&](size_t task) {
            const int m0 = int(task / nt) * 4, n0 = int(task % nt) * 4;
            float acc[4][4] = {};
            const int mm = std::min(4, M - m0), nn = std::min(4, N - n0);
            for (int k = 0; k < K; ++k) {
                float xv[4], wv[4];
                for (int i = 0; i < 4; ++i) xv[i] = i < mm ? Elem<T>::ld(in, size_t(m0 + i) * K + k) : 0.f;
                for (int j = 0; j < 4; ++j) wv[j] = j < nn ? Elem<T>::ld(weight, size_t(n0 + j) * K + k) : 0.f;
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 4; ++j) acc[i][j] += xv[i] * wv[j];
            }
            for (int i = 0; i < mm; ++i)
                for (int j = 0; j < nn; ++j) {
                    float v = acc[i][j];
                    if (bias) v += Elem<T>::ld(bias, n0 + j);
                    Elem<T>::st(out, size_t(m0 + i) * N + n0 + j, v);
                }
        });
    }
};

void linear(void *out, const void *in, const void *weight, const void *bias, ElemType t, int M, int N, int K) {
    if (M == 0 || N == 0) return;
    byType<LinearOp>(t, out, in, weight, bias, M, N, K);
}

void rearrange(void *out, const void *in, size_t esz, int ndim, const int64_t *shape, const int64_t *out_strides,
               const int64_t *in_strides) {
    size_t n = 1;
    for (int k = 0; k < ndim; ++k) n *= size_t(shape[k]);
    auto *o = static_cast<std::byte *>(out);
    const auto *s = static_cast<const std::byte *>(in);
    parallelFor(n, 1 << 14, [&](size_t i) {
        size_t rem = i;
        int64_t oo = 0, io = 0;
        for (int k = ndim - 1; k >= 0; --k) {
            const int64_t c = int64_t(rem % size_t(shape[k]));
            rem /= size_t(shape[k]);
            oo += c * out_strides[k];
            io += c * in_strides[k];
        }
        std::memcpy(o + oo * int64_t(esz), s + io * int64_t(esz), esz);
    });
}

void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType t, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale) {
    if (L == 0) return;
    std::vector<float> Kf(size_t(S) * nkvh * d), Vf(size_t(S) * nkvh * dv);
    widen(Kf.data(), k, t, Kf.size());
    widen(Vf.data(), v, t, Vf.size());
    const int G = nh / nkvh;
    parallelFor(size_t(L) * nh, 1, [&](size_t task) {
        const int i = int(task / nh), h = int(task % nh), hk = h / G;
        thread_local std::vector<float> s, qf, o;
        s.resize(size_t(S));
        qf.resize(size_t(d));
        o.resize(size_t(dv));
        for (int c = 0; c < d; ++c) qf[c] = ldAny(t, q, (size_t(i) * nh + h) * d + c);
        const int n = std::min(S, i + S - L + 1); // keys j <= i + S - L
        attendRow(o.data(), s.data(), qf.data(), Kf.data() + size_t(hk) * d, Vf.data() + size_t(hk) * dv, n, d, dv,
                  size_t(nkvh) * d, size_t(nkvh) * dv, scale, nullptr);
        for (int c = 0; c < dv; ++c) {
            const size_t oi = (size_t(i) * nh + h) * dv + c;
            switch (t) {
            case ElemType::F32: Elem<float>::st(out, oi, o[c]); break;
            case ElemType::F16: Elem<F16>::st(out, oi, o[c]); break;
            case ElemType::BF16: Elem<BF16>::st(out, oi, o[c]); break;
            }
        }
    });
}

void pagedAppend(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                 const int32_t *table, const int32_t *ctx, const int32_t *cu_new, int T, int B, int nkvh,
                 int max_pages, int num_blocks, int *err) {
    parallelFor(size_t(T), 64, [&](size_t r) {
        const int b = cu_new ? owningSequence(cu_new, B, int(r)) : int(r);
        const int pos = cu_new ? ctx[b] + (int(r) - cu_new[b]) : ctx[b];
        const int page = pos >> 4, slot = pos & 15;
        if (pos < 0 || page >= max_pages) {
            raiseFlag(err, kErrTooLong);
            return;
        }
        const int blk = table[size_t(b) * max_pages + page];
        if (blk < 0 || blk >= num_blocks) {
            raiseFlag(err, kErrBadBlock);
            return;
        }
        for (int h = 0; h < nkvh; ++h) {
            const size_t base = (size_t(blk) * nkvh + h) * kPageElems;
            const size_t row = (r * nkvh + h) * kHeadDim;
            for (int dd = 0; dd < kHeadDim; ++dd) {
                k_pool[base + kIndex(slot, dd)] = k_new[row + dd];
                v_pool[base + vIndex(slot, dd)] = v_new[row + dd];
            }
        }
    });
}

namespace {

// Rows [0, n) of one (block, head) page out to row-major rows of stride
// nkvh * 128 elements.
void pageOut(uint16_t *k_dst, uint16_t *v_dst, const uint16_t *kpage, const uint16_t *vpage, int n, int nkvh) {
    for (int t = 0; t < n; ++t) {
        uint16_t *kr = k_dst + size_t(t) * nkvh * kHeadDim;
        uint16_t *vr = v_dst + size_t(t) * nkvh * kHeadDim;
        for (int c = 0; c < kHeadDim / 8; ++c) std::memcpy(kr + c * 8, kpage + c * 128 + t * 8, 16);
        for (int dd = 0; dd < kHeadDim; ++dd) vr[dd] = vpage[vIndex(t, dd)];
    }
}

// One sequence's gather (rows row0.. of k_out/v_out), shared by the plain and
// fused paths. The sequence has already been validated against T.
void gatherSequence(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                    const int32_t *trow, int row0, int len, int nkvh, int max_pages, int num_blocks, int *err) {
    if (len > max_pages * kPageTokens) raiseFlag(err, kErrTooLong);
    const int pages = std::min((len + 15) / 16, max_pages);
    for (int p = 0; p < pages; ++p) {
        const int blk = trow[p];
        if (blk < 0 || blk >= num_blocks) {
            raiseFlag(err, kErrBadBlock);
            continue;
        }
        const int n = std::min(16, len - 16 * p);
        for (int h = 0; h < nkvh; ++h) {
            const size_t base = (size_t(blk) * nkvh + h) * kPageElems;
            const size_t dst = (size_t(row0 + 16 * p) * nkvh + h) * kHeadDim;
            pageOut(k_out + dst, v_out + dst, k_pool + base, v_pool + base, n, nkvh);
        }
    }
}

} // namespace

void pagedGather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *table, const int32_t *cu, int T, int B, int nkvh, int max_pages, int num_blocks,
                 int *err) {
    parallelFor(size_t(B), 1, [&](size_t b) {
        const int row0 = cu[b], len = cu[b + 1] - row0;
        if (len <= 0) return;
        if (row0 < 0 || cu[b + 1] > T) {
            raiseFlag(err, kErrTooLong);
            return;
        }
        gatherSequence(k_out, v_out, k_pool, v_pool, table + b * size_t(max_pages), row0, len, nkvh, max_pages,
                       num_blocks, err);
    });
}

void pagedAppendGather(uint16_t *k_out, uint16_t *v_out, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new,
                       const uint16_t *v_new, const int32_t *table, const int32_t *ctx, const int32_t *cu, int T,
                       int B, int nkvh, int max_pages, int num_blocks, int *err) {
    parallelFor(size_t(B), 1, [&](size_t b) {
        const int c = ctx[b], row0 = cu[b], len = cu[b + 1] - row0;
        if (c < 0 || len != c + 1) {
            raiseFlag(err, kErrTooLong);
            return;
        }
        if (row0 < 0 || cu[b + 1] > T) {
            raiseFlag(err, kErrTooLong);
            return;
        }
        const int32_t *trow = table + b * size_t(max_pages);
        const int page = c >> 4, slot = c & 15;
        if (page < max_pages) {
            const int blk = trow[page];
            if (blk >= 0 && blk < num_blocks) {
                for (int h = 0; h < nkvh; ++h) {
                    const size_t base = (size_t(blk) * nkvh + h) * kPageElems;
                    const size_t row = (b * size_t(nkvh) + h) * kHeadDim;
                    for (int dd = 0; dd < kHeadDim; ++dd) {
                        k_pool[base + kIndex(slot, dd)] = k_new[row + dd];
                        v_pool[base + vIndex(slot, dd)] = v_new[row + dd];
                    }
                }
            }
        }
        gatherSequence(k_out, v_out, k_pool, v_pool, trow, row0, len, nkvh, max_pages, num_blocks, err);
    });
}

void pagedCopyBlocks(uint16_t *k_pool, uint16_t *v_pool, const int32_t *pairs, int P, int nkvh, int num_blocks,
                     int *err) {
    const size_t per_block = size_t(nkvh) * kPageElems;
    // Sequential: a later pair may read a block an earlier one wrote.
    for (int i = 0; i < P; ++i) {
        const int s = pairs[2 * i], d = pairs[2 * i + 1];
        if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) {
            raiseFlag(err, kErrBadBlock);
            continue;
        }
        std::memcpy(k_pool + d * per_block, k_pool + s * per_block, per_block * 2);
        std::memcpy(v_pool + d * per_block, v_pool + s * per_block, per_block * 2);
    }
}

void pagedAttention(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                    const int32_t *table, const int32_t *ctx, const int32_t *cu_q, int B, int T, int nh, int nkvh,
                    int max_pages, int num_blocks, float scale, int *err) {
    const int G = nh / nkvh;
    auto store = [&](size_t row, int h, const float *o) {
        const size_t base = (row * nh + h) * kHeadDim;
        for (int c = 0; c < kHeadDim; ++c) {
            if (out_f32)
                static_cast<float *>(out)[base + c] = o[c];
            else
                static_cast<uint16_t *>(out)[base + c] = f32ToBf16(o[c]);
        }
    };
    parallelFor(size_t(B) * nkvh, 1, [&](size_t task) {
        const int b = int(task / nkvh), hk = int(task % nkvh);
        const int q0 = cu_q ? cu_q[b] : b;
        const int Lq = cu_q ? cu_q[b + 1] - q0 : 1;
        if (Lq <= 0) return;
        const int c = ctx[b];
        float zeros[kHeadDim] = {};
        if (q0 < 0 || q0 + Lq > T || c < Lq || c > max_pages * kPageTokens) {
            if (hk == 0) raiseFlag(err, kErrTooLong);
            if (q0 >= 0 && q0 + Lq <= T)
                for (int i = 0; i < Lq; ++i)
                    for (int g = 0; g < G; ++g) store(size_t(q0 + i), hk * G + g, zeros);
            return;
        }
        // This sequence's K and V of kv head hk, row-major fp32.
        thread_local std::vector<float> K, V, s;
        thread_local std::vector<uint8_t> skip;
        K.resize(size_t(c) * kHeadDim);
        V.resize(size_t(c) * kHeadDim);
        s.resize(size_t(c));
        skip.assign(size_t(c), 0);
        const int32_t *trow = table + size_t(b) * max_pages;
        for (int p = 0; p * 16 < c; ++p) {
            const int blk = trow[p];
            const int n = std::min(16, c - 16 * p);
            if (blk < 0 || blk >= num_blocks) {
                if (hk == 0) raiseFlag(err, kErrBadBlock);
                std::fill(skip.begin() + 16 * p, skip.begin() + 16 * p + n, 1);
                continue;
            }
            const uint16_t *kp = k_pool + (size_t(blk) * nkvh + hk) * kPageElems;
            const uint16_t *vp = v_pool + (size_t(blk) * nkvh + hk) * kPageElems;
            for (int t = 0; t < n; ++t)
                for (int dd = 0; dd < kHeadDim; ++dd) {
                    K[size_t(16 * p + t) * kHeadDim + dd] = bf16ToF32(kp[kIndex(t, dd)]);
                    V[size_t(16 * p + t) * kHeadDim + dd] = bf16ToF32(vp[vIndex(t, dd)]);
                }
        }
        float qf[kHeadDim], o[kHeadDim];
        for (int i = 0; i < Lq; ++i) {
            const int visible = c - Lq + i + 1; // bottom-right causal
            for (int g = 0; g < G; ++g) {
                const int h = hk * G + g;
                const uint16_t *qr = q + (size_t(q0 + i) * nh + h) * kHeadDim;
                for (int dd = 0; dd < kHeadDim; ++dd) qf[dd] = bf16ToF32(qr[dd]);
                attendRow(o, s.data(), qf, K.data(), V.data(), visible, kHeadDim, kHeadDim, kHeadDim, kHeadDim, scale,
                          skip.data());
                store(size_t(q0 + i), h, o);
            }
        }
    });
}

} // namespace llaisys::cpu
