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
