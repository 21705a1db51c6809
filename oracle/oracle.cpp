// TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.
//
// CPU FP64 restatement of the reference's attention oracle and its accuracy
// comparator. Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
// bench.py may load this library, and only as the checker (or, for the CPU
// baseline, as the thing timed on the host). The HIP product path never links
// or calls it.
//
// Each function cites the reference file:line it restates
// (paths relative to the RichterWang/cuda_fused_attention tree):
//
//   bf16_from_float     IEEE-754 round-to-nearest-even fp32 -> bf16, the
//                        semantics of __float2bfloat16 used by
//                        benchmarks/bench_flash_attention.cu:91,211
//   bf16_ulp            benchmarks/bench_flash_attention.cu:95-102
//   default_scale       include/flash_attention.h:21-24
//   attention_flops     kernels/v0_unfused.cu:118-126 (reference convention)
//   workspace bytes     kernels/v0_unfused.cu:128-131
//   fill_normal_mt19937 benchmarks/bench_flash_attention.cu:86-92
//   attention           benchmarks/bench_flash_attention.cu:105-145
//   compare             benchmarks/bench_flash_attention.cu:148-218
//   qkvo / score bytes  benchmarks/bench_flash_attention.cu:221-231
//   v3 traffic model    kernels/v3/v3_tensorcore.cu:795-818
//
// The uniform / Box-Muller generators are this repository's own input
// generators (SplitMix64 stream), documented next to their definitions.
//
// Pins (tests/test_oracle_pins.py): exhaustive bf16 RNE check over all 2^32
// float bit patterns, closed-form special cases (N=1, Q=K=0, all-ones,
// constant V, one-hot logits), an independent numpy long-double brute force,
// the C++-standard mt19937 known answer, and the reference's own published
// accuracy statistics (results/raw/flash_attention/accuracy.csv:2-21).

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <thread>
#include <vector>

namespace {

inline uint32_t float_bits(float x)
{
    uint32_t u;
    std::memcpy(&u, &x, sizeof(u));
    return u;
}

inline float bits_float(uint32_t u)
{
    float x;
    std::memcpy(&x, &u, sizeof(x));
    return x;
}

// Round-to-nearest-even on the upper 16 bits of the IEEE-754 binary32 word.
// NaN stays NaN (quiet bit forced so truncation cannot turn it into Inf);
// overflow past the largest finite bf16 carries into the exponent and gives
// +-Inf, exactly as the IEEE definition of RNE requires.
inline uint16_t rne_bf16(float x)
{
    const uint32_t u = float_bits(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u)
        return static_cast<uint16_t>((u >> 16) | 0x0040u);
    const uint32_t lsb = (u >> 16) & 1u;
    const uint32_t rounded = u + 0x7fffu + lsb;
    return static_cast<uint16_t>(rounded >> 16);
}

inline float bf16_to_float(uint16_t b) { return bits_float(static_cast<uint32_t>(b) << 16); }

// SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014). The seed is the initial state; each call adds
// the golden-ratio increment and mixes.
struct SplitMix64
{
    uint64_t state;
    explicit SplitMix64(uint64_t seed) : state(seed) {}
    uint64_t next()
    {
        uint64_t z = (state += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    // uniform in [0, 1) on the 2^-24 grid (exact in binary32)
    float unit24() { return static_cast<float>(next() >> 40) * 0x1.0p-24f; }
    // uniform in [0, 1) on the 2^-53 grid
    double unit53() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }
};

int pick_threads(int requested, int64_t work_rows)
{
    int threads = requested;
    if (threads <= 0)
    {
        const unsigned hc = std::thread::hardware_concurrency();
        threads = hc == 0 ? 1 : static_cast<int>(hc);
    }
    if (threads > 256) threads = 256;
    if (work_rows < threads) threads = static_cast<int>(std::max<int64_t>(work_rows, 1));
    return threads;
}

// One output row of benchmarks/bench_flash_attention.cu:117-142: FP64 dot
// products of bf16->double inputs, the float scale promoted to double, a
// max-subtracted exp, and the normalised weighted sum.
void oracle_row(const uint16_t* q, const uint16_t* k, const uint16_t* v, double* out_row,
                int n, int d, int query, bool causal, double scale, double* scores)
{
    const int limit = causal ? query + 1 : n;
    const uint16_t* q_row = q + static_cast<size_t>(query) * d;

    double row_max = -1.0e300;
    for (int key = 0; key < limit; ++key)
    {
        const uint16_t* k_row = k + static_cast<size_t>(key) * d;
        double dot = 0.0;
        for (int dim = 0; dim < d; ++dim)
            dot += static_cast<double>(bf16_to_float(q_row[dim])) *
                   static_cast<double>(bf16_to_float(k_row[dim]));
        scores[key] = dot * scale;
        row_max = std::max(row_max, scores[key]);
    }

    double sum = 0.0;
    for (int key = 0; key < limit; ++key)
    {
        scores[key] = std::exp(scores[key] - row_max);
        sum += scores[key];
    }

    for (int dim = 0; dim < d; ++dim) out_row[dim] = 0.0;
    for (int key = 0; key < limit; ++key)
    {
        const uint16_t* v_row = v + static_cast<size_t>(key) * d;
        const double p = scores[key];
        for (int dim = 0; dim < d; ++dim)
            out_row[dim] += p * static_cast<double>(bf16_to_float(v_row[dim]));
    }
    for (int dim = 0; dim < d; ++dim) out_row[dim] /= sum;
}

// ---------------------------------------------------------------------------
// The same arithmetic as oracle_row, reorganised for cache reuse: a group of
// up to kGroup queries of one slab walks the keys in tiles of kKeyTile, with
// register blocks of kQB queries x kKB keys (scores) and kQB queries x kDB
// head dims (P.V). Every score is still the sequential sum over head dims
// 0..D-1 of double(q)*double(k), times the promoted float scale; every output
// element is still the sequential sum over keys 0..limit-1 of p*double(v);
// the max, exp, sum and division run per query in key order. Only the order
// in which independent sums are advanced changes, so each output is
// bitwise identical to oracle_row's (tests/test_oracle_pins.py checks that
// against fa_oracle_attention_scalar). Keys past a query's causal limit are
// never added into its sums.
constexpr int kGroup = 64;     // queries per work item
constexpr int kKeyTile = 256;  // keys per cache tile
constexpr int kQB = 4;         // queries per register block
constexpr int kKB = 8;         // keys per score register block
constexpr int kDB = 8;         // head dims per P.V register block

struct SlabCache
{
    int n_pad = 0;           // seq_len rounded up to kKB
    std::vector<double> kt;  // K^T as double, [head_dim][n_pad], zero padded
    std::vector<double> vd;  // V as double, [seq_len][head_dim]
};

void fill_slab_cache(SlabCache& c, const uint16_t* k, const uint16_t* v, int n, int d)
{
    c.n_pad = (n + kKB - 1) / kKB * kKB;
    c.kt.assign(static_cast<size_t>(d) * c.n_pad, 0.0);
    c.vd.resize(static_cast<size_t>(n) * d);
    for (int key = 0; key < n; ++key)
        for (int dim = 0; dim < d; ++dim)
        {
            c.kt[static_cast<size_t>(dim) * c.n_pad + key] = bf16_to_float(k[static_cast<size_t>(key) * d + dim]);
            c.vd[static_cast<size_t>(key) * d + dim] = bf16_to_float(v[static_cast<size_t>(key) * d + dim]);
        }
}

// Four doubles in one vector (GCC vector extension): AVX2 registers in the
// avx2 clone, SSE2 pairs otherwise. Element-wise + and * are plain IEEE
// double operations (the build uses -ffp-contract=off: no fused forms).
typedef double v4d __attribute__((vector_size(32)));

__attribute__((always_inline)) inline v4d load4(const double* p)
{
    v4d x;
    std::memcpy(&x, p, sizeof(x));
    return x;
}

__attribute__((always_inline)) inline void store4(double* p, v4d x) { std::memcpy(p, &x, sizeof(x)); }

// Scores of kQB queries (qd: [kQB][d] doubles) against keys [key0, key1),
// key1 - key0 a multiple of kKB, into sc[t * stride + key]. Vector lane j of
// acc[t][h] is the running dot product of query t with key kb + 4h + j,
// summed over head dims in increasing order.
__attribute__((target_clones("avx2", "default"))) void score_block(const double* qd, const double* kt, int n_pad,
                                                                   int d, int key0, int key1, double scale,
                                                                   double* sc, int stride)
{
    static_assert(kKB == 8, "two vectors of keys per register block");
    for (int kb = key0; kb < key1; kb += kKB)
    {
        v4d acc[kQB][2] = {};
        for (int dim = 0; dim < d; ++dim)
        {
            const double* kr = kt + static_cast<size_t>(dim) * n_pad + kb;
            const v4d k0 = load4(kr);
            const v4d k1 = load4(kr + 4);
            for (int t = 0; t < kQB; ++t)
            {
                const v4d qv = v4d{} + qd[t * d + dim];
                acc[t][0] += qv * k0;
                acc[t][1] += qv * k1;
            }
        }
        for (int t = 0; t < kQB; ++t)
        {
            store4(sc + static_cast<size_t>(t) * stride + kb, acc[t][0] * scale);
            store4(sc + static_cast<size_t>(t) * stride + kb + 4, acc[t][1] * scale);
        }
    }
}

// out[t][dim] += sum over keys [key0, key1) of p[t][key] * v[key][dim] for
// kQB queries, keys in increasing order, every dim block of kDB.
__attribute__((target_clones("avx2", "default"))) void pv_block4(const double* p, int stride, const double* vd,
                                                                 int d, int key0, int key1, double* out)
{
    const int d_full = d / kDB * kDB;
    for (int d0 = d_full; d0 < d; ++d0)  // head dims past the last full block
        for (int key = key0; key < key1; ++key)
            for (int t = 0; t < kQB; ++t)
                out[t * d + d0] += p[static_cast<size_t>(t) * stride + key] * vd[static_cast<size_t>(key) * d + d0];
    static_assert(kDB == 8, "two vectors of head dims per register block");
    for (int d0 = 0; d0 < d_full; d0 += kDB)
    {
        v4d acc[kQB][2];
        for (int t = 0; t < kQB; ++t)
        {
            acc[t][0] = load4(out + t * d + d0);
            acc[t][1] = load4(out + t * d + d0 + 4);
        }
        for (int key = key0; key < key1; ++key)
        {
            const double* vr = vd + static_cast<size_t>(key) * d + d0;
            const v4d v0 = load4(vr);
            const v4d v1 = load4(vr + 4);
            for (int t = 0; t < kQB; ++t)
            {
                const v4d pv = v4d{} + p[static_cast<size_t>(t) * stride + key];
                acc[t][0] += pv * v0;
                acc[t][1] += pv * v1;
            }
        }
        for (int t = 0; t < kQB; ++t)
        {
            store4(out + t * d + d0, acc[t][0]);
            store4(out + t * d + d0 + 4, acc[t][1]);
        }
    }
}

// One query's share of keys [key0, key1) (the keys past the smallest causal
// limit of its register block), same order.
void pv_row(const double* p, const double* vd, int d, int key0, int key1, double* out)
{
    for (int key = key0; key < key1; ++key)
    {
        const double pv = p[key];
        const double* vr = vd + static_cast<size_t>(key) * d;
        for (int dim = 0; dim < d; ++dim) out[dim] += pv * vr[dim];
    }
}

// A group of queries of one slab (q: the slab's Q, queries[i] its query
// indices, any order); out_rows[i] receives query i's output row.
void oracle_group(const uint16_t* q, const SlabCache& c, int n, int d, const int* queries, int count, bool causal,
                  double scale, double* const* out_rows, std::vector<double>& scores, std::vector<double>& qd,
                  std::vector<double>& acc)
{
    const int blocks = (count + kQB - 1) / kQB;
    const int rows = blocks * kQB;  // padded with copies of the last query
    const int stride = c.n_pad;
    scores.resize(static_cast<size_t>(rows) * stride);
    qd.resize(static_cast<size_t>(rows) * d);
    acc.assign(static_cast<size_t>(rows) * d, 0.0);
    std::vector<int> qi(static_cast<size_t>(rows)), lim(static_cast<size_t>(rows));
    int max_lim = 0;
    for (int t = 0; t < rows; ++t)
    {
        qi[t] = queries[std::min(t, count - 1)];
        lim[t] = causal ? qi[t] + 1 : n;
        max_lim = std::max(max_lim, lim[t]);
        for (int dim = 0; dim < d; ++dim)
            qd[static_cast<size_t>(t) * d + dim] = bf16_to_float(q[static_cast<size_t>(qi[t]) * d + dim]);
    }

    // Scores, key tile by key tile (a tile of K^T stays in cache for the group).
    for (int k0 = 0; k0 < max_lim; k0 += kKeyTile)
        for (int b = 0; b < blocks; ++b)
        {
            int blim = 0;
            for (int t = b * kQB; t < b * kQB + kQB; ++t) blim = std::max(blim, lim[t]);
            const int k1 = std::min(k0 + kKeyTile, (blim + kKB - 1) / kKB * kKB);
            if (k1 > k0)
                score_block(&qd[static_cast<size_t>(b) * kQB * d], c.kt.data(), c.n_pad, d, k0, k1, scale,
                            &scores[static_cast<size_t>(b) * kQB * stride], stride);
        }

    // Row max, exp and sum per query over its own keys, in key order.
    std::vector<double> sums(static_cast<size_t>(rows));
    for (int t = 0; t < rows; ++t)
    {
        double* sc = &scores[static_cast<size_t>(t) * stride];
        double row_max = -1.0e300;
        for (int key = 0; key < lim[t]; ++key) row_max = std::max(row_max, sc[key]);
        double sum = 0.0;
        for (int key = 0; key < lim[t]; ++key)
        {
            sc[key] = std::exp(sc[key] - row_max);
            sum += sc[key];
        }
        sums[t] = sum;
    }

    // P.V: the keys every query of a register block sees go through the
    // blocked kernel, each query's remaining keys through pv_row, tile by
    // tile, so every sum still runs over keys in increasing order.
    for (int k0 = 0; k0 < max_lim; k0 += kKeyTile)
        for (int b = 0; b < blocks; ++b)
        {
            int bmin = n, bmax = 0;
            for (int t = b * kQB; t < b * kQB + kQB; ++t)
            {
                bmin = std::min(bmin, lim[t]);
                bmax = std::max(bmax, lim[t]);
            }
            const int k1 = std::min(k0 + kKeyTile, bmax);
            if (k1 <= k0) continue;
            const int common = std::min(k1, bmin);
            if (common > k0)
                pv_block4(&scores[static_cast<size_t>(b) * kQB * stride], stride, c.vd.data(), d, k0, common,
                          &acc[static_cast<size_t>(b) * kQB * d]);
            for (int t = b * kQB; t < b * kQB + kQB; ++t)
            {
                const int lo = std::max(k0, common);
                const int hi = std::min(k1, lim[t]);
                if (hi > lo)
                    pv_row(&scores[static_cast<size_t>(t) * stride], c.vd.data(), d, lo, hi,
                           &acc[static_cast<size_t>(t) * d]);
            }
        }

    for (int t = 0; t < count; ++t)
        for (int dim = 0; dim < d; ++dim) out_rows[t][dim] = acc[static_cast<size_t>(t) * d + dim] / sums[t];
}

}  // namespace

extern "C" {

// Accuracy record: benchmarks/bench_flash_attention.cu:148-164, plus the
// BASELINE tolerance |O - O_ref| <= 2^-7 * max|O_ref row| as `abs_gate`
// (the largest value of |err| / (2^-7 * row_scale) seen; passes when <= 1).
struct fa_oracle_accuracy
{
    double vs_double;
    double row_scaled;
    double max_abs;
    double ulp;
    double abs_gate;
    int64_t output_nan;
    int64_t output_inf;
    int64_t reference_nan;
    int64_t reference_inf;
    int32_t passed_ulp;   // reference's Accuracy::passed(): finite and ulp <= 2
    int32_t passed_abs;   // finite and abs_gate <= 1
};

uint16_t fa_oracle_bf16_from_float(float x) { return rne_bf16(x); }

float fa_oracle_float_from_bf16(uint16_t b) { return bf16_to_float(b); }

void fa_oracle_bf16_from_float_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = rne_bf16(in[i]);
}

// Independent restatement used to pin rne_bf16 exhaustively: pick the nearer
// of the two bf16 neighbours of x by exact arithmetic on the discarded bits,
// ties to the even mantissa. Covers finite values and infinities; NaN is
// handled by the caller's check.
uint16_t fa_oracle_bf16_from_float_slow(float x)
{
    const uint32_t u = float_bits(x);
    const uint32_t sign = u & 0x80000000u;
    const uint32_t mag = u & 0x7fffffffu;
    if (mag > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);  // NaN
    const uint32_t down = mag & 0xffff0000u;   // truncation toward zero
    const uint32_t rest = mag & 0x0000ffffu;   // discarded magnitude bits
    uint32_t chosen;
    if (rest < 0x8000u) chosen = down;
    else if (rest > 0x8000u) chosen = down + 0x10000u;
    else chosen = ((down >> 16) & 1u) ? down + 0x10000u : down;  // tie: keep even
    return static_cast<uint16_t>((sign | chosen) >> 16);
}

// benchmarks/bench_flash_attention.cu:95-102
float fa_oracle_bf16_ulp(float value)
{
    if (value == 0.0f || !std::isfinite(value)) return std::ldexp(1.0f, -126 - 7);
    int exponent = 0;
    std::frexp(std::fabs(value), &exponent);
    return std::ldexp(1.0f, std::max(exponent - 8, -133));
}

// include/flash_attention.h:21-24
float fa_oracle_default_scale(int head_dim) { return 1.0f / std::sqrt(static_cast<float>(head_dim)); }

// kernels/v0_unfused.cu:118-126 (causal pairs N(N+1)/2)
double fa_oracle_attention_flops(int batch, int heads, int seq_len, int head_dim, int causal)
{
    const double n = static_cast<double>(seq_len);
    const double pairs = causal ? n * (n + 1.0) / 2.0 : n * n;
    return 4.0 * pairs * head_dim * static_cast<double>(batch) * heads;
}

// kernels/v0_unfused.cu:128-131
uint64_t fa_oracle_unfused_workspace_bytes(int batch, int heads, int seq_len)
{
    return static_cast<uint64_t>(batch) * heads * seq_len * seq_len * sizeof(float);
}

// benchmarks/bench_flash_attention.cu:221-231
double fa_oracle_qkvo_bytes(int batch, int heads, int seq_len, int head_dim)
{
    return 4.0 * batch * heads * static_cast<double>(seq_len) * head_dim * 2.0;
}

double fa_oracle_unfused_score_bytes(int batch, int heads, int seq_len)
{
    return 5.0 * batch * heads * static_cast<double>(seq_len) * seq_len * sizeof(float);
}

// kernels/v3/v3_tensorcore.cu:795-818: Q read once, O written once, and the
// K/V tiles counted per query block that loads them (whole tiles).
double fa_oracle_blocked_kv_hbm_bytes(int batch, int heads, int seq_len, int head_dim,
                                      int causal, int rows_per_block, int tile_kv)
{
    const double element = 2.0;
    const int slabs = batch * heads;
    const int row_blocks = (seq_len + rows_per_block - 1) / rows_per_block;
    double bytes = 2.0 * slabs * static_cast<double>(seq_len) * head_dim * element;
    double kv_tiles = 0.0;
    for (int block = 0; block < row_blocks; ++block)
    {
        const int q_max = block * rows_per_block + rows_per_block - 1;
        const int key_limit = causal ? std::min(q_max, seq_len - 1) : seq_len - 1;
        kv_tiles += static_cast<double>((key_limit + tile_kv) / tile_kv);
    }
    bytes += 2.0 * slabs * kv_tiles * tile_kv * head_dim * element;
    return bytes;
}

// This repository's uniform[-1,1) input family: SplitMix64(seed), top 24 bits
// -> u in [0,1) exactly, x = 2u - 1 (exact), then RNE to bf16.
void fa_oracle_fill_uniform(uint16_t* out, int64_t n, uint64_t seed)
{
    SplitMix64 rng(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = rne_bf16(2.0f * rng.unit24() - 1.0f);
}

// This repository's N(0, sigma^2) family: Box-Muller on the same stream,
// z = sqrt(-2 ln(1-u1)) * cos(2 pi u2) in double, scaled, rounded to float,
// then RNE to bf16. One pair of draws per output element.
void fa_oracle_fill_normal(uint16_t* out, int64_t n, uint64_t seed, double sigma)
{
    SplitMix64 rng(seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; ++i)
    {
        const double u1 = rng.unit53();
        const double u2 = rng.unit53();
        const double radius = std::sqrt(-2.0 * std::log1p(-u1));
        out[i] = rne_bf16(static_cast<float>(sigma * radius * std::cos(two_pi * u2)));
    }
}

// benchmarks/bench_flash_attention.cu:86-92: std::mt19937(seed) feeding
// std::normal_distribution<float>(0,1), each draw rounded to bf16 (RNE).
// Reproduces the reference's inputs bit-for-bit with the same standard
// library family (libstdc++).
void fa_oracle_fill_normal_mt19937(uint16_t* out, int64_t n, uint32_t seed)
{
    std::mt19937 engine(seed);
    std::normal_distribution<float> dist(0.0f, 1.0f);
    for (int64_t i = 0; i < n; ++i) out[i] = rne_bf16(dist(engine));
}

// The 10000th output of a default-constructed std::mt19937 (C++ standard,
// [rand.predef]: 4123659995). Lets a test pin the engine the generator above
// is built on.
uint32_t fa_oracle_mt19937_10000th(void)
{
    std::mt19937 engine;
    engine.discard(9999);
    return static_cast<uint32_t>(engine());
}

// benchmarks/bench_flash_attention.cu:105-145, restated.
// q, k, v: bf16 bit patterns, contiguous [batch, heads, seq_len, head_dim].
// rows:    optional list of global row ids r = bh*seq_len + query; when null
//          every row is computed and out is [batch*heads*seq_len, head_dim];
//          otherwise out is [n_rows, head_dim] in the order given.
// threads: <=0 uses std::thread::hardware_concurrency().
// Returns 0, or -1 on an invalid argument.
//
// The rows are grouped by slab and computed by oracle_group (the blocked
// form of oracle_row, bitwise identical to it); fa_oracle_attention_scalar
// below runs oracle_row itself, one row at a time.
int fa_oracle_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, double* out,
                        int batch, int heads, int seq_len, int head_dim, int causal,
                        const int64_t* rows, int64_t n_rows, int threads)
{
    if (batch < 0 || heads < 0 || seq_len < 0 || head_dim <= 0) return -1;
    const int64_t total_rows = static_cast<int64_t>(batch) * heads * seq_len;
    const int64_t work = rows ? n_rows : total_rows;
    if (work <= 0) return 0;
    if (rows)
        for (int64_t i = 0; i < n_rows; ++i)
            if (rows[i] < 0 || rows[i] >= total_rows) return -1;

    const double scale = static_cast<double>(fa_oracle_default_scale(head_dim));
    const int64_t slabs = static_cast<int64_t>(batch) * heads;

    // Output positions ordered by (slab, query): slab s owns order[first[s] .. first[s+1]).
    std::vector<int64_t> order(static_cast<size_t>(work));
    for (int64_t i = 0; i < work; ++i) order[static_cast<size_t>(i)] = i;
    auto row_of = [&](int64_t i) { return rows ? rows[i] : i; };
    if (rows)
        std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return row_of(a) < row_of(b); });
    std::vector<int64_t> first(static_cast<size_t>(slabs) + 1, 0);
    for (int64_t i = 0; i < work; ++i) ++first[static_cast<size_t>(row_of(i) / seq_len) + 1];
    for (int64_t s = 0; s < slabs; ++s) first[static_cast<size_t>(s) + 1] += first[static_cast<size_t>(s)];

    // Work items: up to kGroup rows of one slab; small per-slab row counts
    // use smaller groups so every thread gets work.
    const int nthreads = pick_threads(threads, work);
    struct Item
    {
        int64_t slab, begin, end;
    };
    std::vector<Item> items;
    std::vector<int64_t> used;
    for (int64_t s = 0; s < slabs; ++s)
    {
        const int64_t b = first[static_cast<size_t>(s)], e = first[static_cast<size_t>(s) + 1];
        if (e == b) continue;
        used.push_back(s);
        const int64_t per = std::max<int64_t>(kQB, std::min<int64_t>(kGroup, (e - b) / nthreads + 1));
        for (int64_t x = b; x < e; x += per) items.push_back(Item{s, x, std::min(e, x + per)});
    }
    std::vector<SlabCache> cache(static_cast<size_t>(slabs));

    auto run_pool = [&](size_t count, auto&& fn) {
        std::atomic<size_t> next{0};
        auto worker = [&] {
            for (size_t it = next++; it < count; it = next++) fn(it);
        };
        const int t = static_cast<int>(std::min<size_t>(static_cast<size_t>(nthreads), count));
        std::vector<std::thread> pool;
        for (int i = 1; i < t; ++i) pool.emplace_back(worker);
        worker();
        for (auto& th : pool) th.join();
    };

    const size_t slab_elems = static_cast<size_t>(seq_len) * head_dim;
    run_pool(used.size(), [&](size_t u) {
        const int64_t s = used[u];
        fill_slab_cache(cache[static_cast<size_t>(s)], k + static_cast<size_t>(s) * slab_elems,
                        v + static_cast<size_t>(s) * slab_elems, seq_len, head_dim);
    });
    run_pool(items.size(), [&](size_t it) {
        thread_local std::vector<double> scores, qd, acc;
        const Item& item = items[it];
        std::vector<int> queries;
        std::vector<double*> dst;
        for (int64_t x = item.begin; x < item.end; ++x)
        {
            const int64_t i = order[static_cast<size_t>(x)];
            queries.push_back(static_cast<int>(row_of(i) % seq_len));
            dst.push_back(out + static_cast<size_t>(i) * head_dim);
        }
        oracle_group(q + static_cast<size_t>(item.slab) * slab_elems, cache[static_cast<size_t>(item.slab)],
                     seq_len, head_dim, queries.data(), static_cast<int>(queries.size()), causal != 0, scale,
                     dst.data(), scores, qd, acc);
    });
    return 0;
}

// The same contract as fa_oracle_attention, computed row by row with
// oracle_row (the direct restatement of bench_flash_attention.cu:117-142).
// Kept as the pin of the blocked path: both must agree bit for bit.
int fa_oracle_attention_scalar(const uint16_t* q, const uint16_t* k, const uint16_t* v, double* out,
                               int batch, int heads, int seq_len, int head_dim, int causal,
                               const int64_t* rows, int64_t n_rows, int threads)
{
    if (batch < 0 || heads < 0 || seq_len < 0 || head_dim <= 0) return -1;
    const int64_t total_rows = static_cast<int64_t>(batch) * heads * seq_len;
    const int64_t work = rows ? n_rows : total_rows;
    if (work <= 0) return 0;
    if (rows)
        for (int64_t i = 0; i < n_rows; ++i)
            if (rows[i] < 0 || rows[i] >= total_rows) return -1;

    const double scale = static_cast<double>(fa_oracle_default_scale(head_dim));
    const int nthreads = pick_threads(threads, work);

    auto body = [&](int64_t begin, int64_t end) {
        std::vector<double> scores(static_cast<size_t>(seq_len));
        for (int64_t i = begin; i < end; ++i)
        {
            const int64_t r = rows ? rows[i] : i;
            const int64_t bh = r / seq_len;
            const int query = static_cast<int>(r % seq_len);
            const size_t slab = static_cast<size_t>(bh) * seq_len * head_dim;
            oracle_row(q + slab, k + slab, v + slab, out + static_cast<size_t>(i) * head_dim,
                       seq_len, head_dim, query, causal != 0, scale, scores.data());
        }
    };

    if (nthreads == 1)
    {
        body(0, work);
        return 0;
    }
    std::vector<std::thread> pool;
    pool.reserve(nthreads);
    // Interleave chunks so causal rows (whose cost grows with the query index)
    // spread evenly over threads.
    const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(64, work / (nthreads * 8) + 1));
    std::vector<int64_t> starts;
    for (int64_t s = 0; s < work; s += chunk) starts.push_back(s);
    for (int t = 0; t < nthreads; ++t)
    {
        pool.emplace_back([&, t] {
            for (size_t c = static_cast<size_t>(t); c < starts.size(); c += static_cast<size_t>(nthreads))
                body(starts[c], std::min(work, starts[c] + chunk));
        });
    }
    for (auto& th : pool) th.join();
    return 0;
}

// benchmarks/bench_flash_attention.cu:167-218, restated, over n_rows rows of
// head_dim values (got: bf16 bit patterns, ref: FP64, same row order).
void fa_oracle_compare(const uint16_t* got, const double* ref, int64_t n_rows, int head_dim,
                       fa_oracle_accuracy* result)
{
    fa_oracle_accuracy acc{};
    const double kRowScaleFloor = 1.0e-6;
    const double gate_unit = std::ldexp(1.0, -7);
    const double inf = std::numeric_limits<double>::infinity();

    for (int64_t row = 0; row < n_rows; ++row)
    {
        const size_t base = static_cast<size_t>(row) * head_dim;
        double row_scale = 0.0;
        for (int dim = 0; dim < head_dim; ++dim)
            if (std::isfinite(ref[base + dim])) row_scale = std::max(row_scale, std::fabs(ref[base + dim]));
        const float scale_ulp = fa_oracle_bf16_ulp(static_cast<float>(row_scale));

        for (int dim = 0; dim < head_dim; ++dim)
        {
            const float g = bf16_to_float(got[base + dim]);
            const double want = ref[base + dim];
            acc.output_nan += std::isnan(g);
            acc.output_inf += std::isinf(g);
            acc.reference_nan += std::isnan(want);
            acc.reference_inf += std::isinf(want);
            if (!std::isfinite(g) || !std::isfinite(want))
            {
                acc.vs_double = acc.row_scaled = acc.max_abs = acc.ulp = acc.abs_gate = inf;
                continue;
            }
            const double abs_error = std::fabs(static_cast<double>(g) - want);
            acc.vs_double = std::max(acc.vs_double, abs_error / std::max(std::fabs(want), 1.0e-6));
            acc.max_abs = std::max(acc.max_abs, abs_error);
            acc.row_scaled = std::max(acc.row_scaled, abs_error / std::max(row_scale, kRowScaleFloor));
            const float rounded = bf16_to_float(rne_bf16(static_cast<float>(want)));
            acc.ulp = std::max(acc.ulp, std::fabs(static_cast<double>(g) - rounded) / scale_ulp);
            const double gate_den = gate_unit * std::max(row_scale, kRowScaleFloor);
            acc.abs_gate = std::max(acc.abs_gate, abs_error / gate_den);
        }
    }
    const bool finite = acc.output_nan == 0 && acc.output_inf == 0 && acc.reference_nan == 0 &&
                        acc.reference_inf == 0;
    acc.passed_ulp = finite && std::isfinite(acc.ulp) && acc.ulp <= 2.0;
    acc.passed_abs = finite && std::isfinite(acc.abs_gate) && acc.abs_gate <= 1.0;
    *result = acc;
}

// Raw SplitMix64 outputs, so a test can pin the generator against its
// published first output for seed 0 (0xe220a8397b1dcdaf).
void fa_oracle_splitmix64(uint64_t seed, uint64_t* out, int64_t n)
{
    SplitMix64 rng(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = rng.next();
}

// Exhaustive pin of rne_bf16: every one of the 2^32 float bit patterns is
// rounded by the bit-trick path and by the slow comparison path
// (fa_oracle_bf16_from_float_slow); returns the number of disagreements.
uint64_t fa_oracle_rne_exhaustive_mismatches(int threads)
{
    const int nthreads = pick_threads(threads, 1 << 20);
    std::vector<uint64_t> bad(static_cast<size_t>(nthreads), 0);
    std::vector<std::thread> pool;
    const uint64_t span = (1ull << 32) / static_cast<uint64_t>(nthreads) + 1;
    for (int t = 0; t < nthreads; ++t)
    {
        pool.emplace_back([&, t] {
            const uint64_t begin = span * static_cast<uint64_t>(t);
            const uint64_t end = std::min<uint64_t>(1ull << 32, begin + span);
            uint64_t count = 0;
            for (uint64_t u = begin; u < end; ++u)
            {
                const float x = bits_float(static_cast<uint32_t>(u));
                count += rne_bf16(x) != fa_oracle_bf16_from_float_slow(x);
            }
            bad[static_cast<size_t>(t)] = count;
        });
    }
    for (auto& th : pool) th.join();
    uint64_t total = 0;
    for (uint64_t b : bad) total += b;
    return total;
}

// Type-7 quantile of an ascending array (benchmarks/bench_flash_attention.cu:243-249).
double fa_oracle_quantile_sorted(const double* sorted, int64_t n, double p)
{
    if (n <= 0) return std::numeric_limits<double>::quiet_NaN();
    const double index = static_cast<double>(n - 1) * p;
    const int64_t lo = static_cast<int64_t>(index);
    const int64_t hi = std::min<int64_t>(lo + 1, n - 1);
    return sorted[lo] + (sorted[hi] - sorted[lo]) * (index - static_cast<double>(lo));
}

}  // extern "C"
