// Correctness and timing harness for libfa_mi355x, written the way a harness
// for the reference is written: it includes only include/flash_attention.h,
// calls cuda_op_lab::flash_attention::* through an entry table, and links
// the library. It restates the study harness of the reference
// (benchmarks/bench_flash_attention.cu:391-731) for HIP:
//   * an accuracy suite on (1,2,256) x head_dim {64,128} x {dense, causal}
//     with the reference's own inputs (std::mt19937 + normal<float>, seeds
//     11/22/33, :86-92) checked by the FP64 oracle;
//   * a timed grid (5 warmups + 30 individually event-timed launches per
//     kernel, median and IQR from type-7 quantiles, :243-299) over BASELINE's
//     grid B {1,2,4} x N {512..8192} x D {64,128} x {dense, causal}, H = 8,
//     uniform[-1,1) inputs reseeded per shape;
//   * the reference's three CSV files (raw_timings.csv, summary.csv,
//     accuracy.csv, :419-424) with its column sets; accuracy.csv adds
//     BASELINE's gate (abs_gate <= 1: |O - O_ref| <= 2^-7 max|O_ref row|).
// Test infrastructure: the FP64 oracle (oracle/liboracle.so) is the checker.
//
// Usage: bench_flash_attention [--quick | --accuracy-only] [--workspace-cap=BYTES] [output_directory]
//        bench_flash_attention --v0-profile [--check] [output_directory]
//        bench_flash_attention --v0-profile B H N D causal [samples [warmup]] [output_directory]
//        bench_flash_attention --v0-profile --profiler B H N D causal [iterations]
//   --quick          B = 1, N in {512, 2048} only (eight grid cases).
//   --accuracy-only  the accuracy suite alone (the ctest).
//   --workspace-cap=BYTES  treat a grid case's v0 workspace above BYTES as
//                    an allocation failure (the reference's out-of-memory
//                    path: v0 SKIP "workspace_allocation_failed", the run
//                    goes on).
//   --v0-profile     the v0 stage profile (benchmarks/profile_attention_v0.cu):
//                    the instrumented launch must equal the plain one bit for
//                    bit (with events, on a non-default stream, and without
//                    events); then, at the reference's two profiling shapes,
//                    30 samples (5 warmups) of the per-stage times (QK,
//                    softmax, PV), the instrumented pipeline and an
//                    unmarked v0 launch, written as v0_stage_timing.csv with
//                    the reference's columns. With --check: the bitwise
//                    checks alone, at N in {1, 17, 256}, D in {64, 128},
//                    dense and causal. With a shape: that shape alone (its
//                    samples and warmups as given, 30 and 5 by default).
//                    With --profiler and a shape: only `iterations` (default
//                    1) instrumented launches without events, no check and no
//                    warmup, for a profiler run (rocprofv3 --kernel-trace
//                    sees one QK, softmax and PV kernel per iteration; the
//                    reference's --ncu mode, profile_attention_v0.cu:195-197).
// Exit status: 0 when every accuracy row passes both gates and every timed
// output is finite, 1 otherwise, 2 on a usage or HIP error.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <iomanip>
#include <locale>
#include <string>
#include <vector>

#include "fa_mi355x.h"
#include "flash_attention.h"
#include "flash_attention_v0_profile.h"
#include "oracle.h"

namespace fa = cuda_op_lab::flash_attention;

namespace {

constexpr int kWarmup = 5;
constexpr int kTimed = 30;

#define HIP_OK(expr)                                                                                       \
    do                                                                                                     \
    {                                                                                                      \
        const hipError_t status_ = (expr);                                                                 \
        if (status_ != hipSuccess)                                                                         \
        {                                                                                                  \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(status_), __FILE__, __LINE__); \
            std::exit(2);                                                                                  \
        }                                                                                                  \
    } while (0)

// One device allocation, freed on scope exit.
struct DeviceBuffer
{
    void* ptr = nullptr;
    size_t bytes = 0;
    explicit DeviceBuffer(size_t n) : bytes(n) { HIP_OK(hipMalloc(&ptr, n)); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer()
    {
        if (ptr) (void)hipFree(ptr);
    }
    __hip_bfloat16* bf16() const { return static_cast<__hip_bfloat16*>(ptr); }
};

struct Problem
{
    const __hip_bfloat16* q;
    const __hip_bfloat16* k;
    const __hip_bfloat16* v;
    __hip_bfloat16* o;
    float* workspace;  // v0 only; may be null when its allocation failed
    fa::AttentionShape shape;
    bool causal;
};

// The harness's kernel table (the reference's kEntries, :342-387, plus the
// v3b slot). Unsupported entries print SKIP, as in the reference.
struct Entry
{
    const char* name;
    std::function<void(const Problem&)> launch;
    std::function<bool(int)> supported;
    std::function<double(const fa::AttentionShape&, bool)> hbm_bytes;  // algorithmic model
    bool needs_workspace;
};

double qkvo_bytes(const fa::AttentionShape& s)
{
    return 4.0 * s.batch * s.heads * static_cast<double>(s.seq_len) * s.head_dim * 2.0;
}

std::vector<Entry> entries()
{
    return {
        {"v0_unfused",
         [](const Problem& p) { fa::launch_attention_unfused(p.q, p.k, p.v, p.o, p.workspace, p.shape, p.causal); },
         [](int) { return true; },
         // the reference's model: five fp32 passes over S (:221-231)
         [](const fa::AttentionShape& s, bool) {
             return qkvo_bytes(s) + 20.0 * s.batch * s.heads * static_cast<double>(s.seq_len) * s.seq_len;
         },
         true},
        {"v1_fused_row",
         [](const Problem& p) { fa::launch_attention_fused_row(p.q, p.k, p.v, p.o, p.shape, p.causal); },
         [](int d) { return fa::fused_row_supported(d); },
         [](const fa::AttentionShape&, bool) { return 0.0; }, false},
        {"v2a_fused_tiled",
         [](const Problem& p) { fa::launch_attention_fusedtiling(p.q, p.k, p.v, p.o, p.shape, p.causal); },
         [](int d) { return fa::query_fused_tiling(d).supported; },
         [](const fa::AttentionShape& s, bool c) { return fa::fused_tiling_hbm_bytes(s, c); }, false},
        {"v2b_fused_tiled",
         [](const Problem& p) { fa::launch_attention_fusedtiling_v2b(p.q, p.k, p.v, p.o, p.shape, p.causal); },
         [](int d) { return fa::query_fused_tiling_v2b(d).supported; },
         [](const fa::AttentionShape& s, bool c) { return fa::fused_tiling_v2b_hbm_bytes(s, c); }, false},
        {"v3_tensorcore",
         [](const Problem& p) { fa::launch_attention_tensorcore_v3(p.q, p.k, p.v, p.o, p.shape, p.causal); },
         [](int d) { return fa::tensorcore_v3_supported(d); },
         [](const fa::AttentionShape& s, bool c) { return fa::tensorcore_v3_hbm_bytes(s, c); }, false},
        {"v3b_tensorcore",
         [](const Problem& p) { fa::launch_attention_tensorcore_v3b(p.q, p.k, p.v, p.o, p.shape, p.causal); },
         [](int d) { return fa::tensorcore_v3b_supported(d); },
         [](const fa::AttentionShape& s, bool c) { return fa::tensorcore_v3b_hbm_bytes(s, c); }, false},
    };
}

size_t elements(const fa::AttentionShape& s)
{
    return static_cast<size_t>(s.batch) * s.heads * s.seq_len * s.head_dim;
}

// bf16 bit patterns with an all-ones exponent are NaN or Inf.
void count_nonfinite(const std::vector<uint16_t>& bits, size_t& nan, size_t& inf)
{
    nan = inf = 0;
    for (uint16_t b : bits)
        if ((b & 0x7f80u) == 0x7f80u) ((b & 0x007fu) ? nan : inf) += 1;
}

struct Summary
{
    std::vector<double> raw;
    double median = 0, q1 = 0, q3 = 0;
};

// Each sample brackets one launch (all of v0's kernels) with events on the
// null stream and waits for it, as the reference's time_iterations does.
Summary time_entry(const Entry& e, const Problem& p)
{
    for (int i = 0; i < kWarmup; ++i) e.launch(p);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
    hipEvent_t start, stop;
    HIP_OK(hipEventCreate(&start));
    HIP_OK(hipEventCreate(&stop));
    Summary s;
    for (int i = 0; i < kTimed; ++i)
    {
        HIP_OK(hipEventRecord(start, nullptr));
        e.launch(p);
        HIP_OK(hipEventRecord(stop, nullptr));
        HIP_OK(hipGetLastError());
        HIP_OK(hipEventSynchronize(stop));
        float ms = 0.0f;
        HIP_OK(hipEventElapsedTime(&ms, start, stop));
        if (!std::isfinite(ms) || ms <= 0.0f)
        {
            std::fprintf(stderr, "invalid event timing %g ms\n", ms);
            std::exit(2);
        }
        s.raw.push_back(ms);
    }
    HIP_OK(hipEventDestroy(start));
    HIP_OK(hipEventDestroy(stop));
    std::vector<double> sorted = s.raw;
    std::sort(sorted.begin(), sorted.end());
    s.median = fa_oracle_quantile_sorted(sorted.data(), static_cast<int64_t>(sorted.size()), 0.5);
    s.q1 = fa_oracle_quantile_sorted(sorted.data(), static_cast<int64_t>(sorted.size()), 0.25);
    s.q3 = fa_oracle_quantile_sorted(sorted.data(), static_cast<int64_t>(sorted.size()), 0.75);
    return s;
}

std::ofstream open_csv(const std::filesystem::path& path, const char* header)
{
    std::ofstream f(path);
    if (!f)
    {
        std::fprintf(stderr, "cannot open %s\n", path.string().c_str());
        std::exit(2);
    }
    f.imbue(std::locale::classic());
    f << std::setprecision(17) << header << '\n';
    return f;
}

void key(std::ostream& f, const char* name, const fa::AttentionShape& s, bool causal)
{
    f << name << ',' << s.batch << ',' << s.heads << ',' << s.seq_len << ',' << s.head_dim << ',' << (causal ? 1 : 0);
}

// Per-shape seeds of the grid, the same as tests/test_gpu_grid.py uses.
uint64_t grid_seed(uint64_t tensor_seed, const fa::AttentionShape& s)
{
    return tensor_seed + 1000ull * s.batch + 10ull * (s.seq_len / 512) + s.head_dim;
}

double quantile_of(std::vector<double> xs, double p)
{
    std::sort(xs.begin(), xs.end());
    return fa_oracle_quantile_sorted(xs.data(), static_cast<int64_t>(xs.size()), p);
}

// One v0 stage-profile shape: bitwise check of the instrumented launch
// against the plain one, then (unless check_only) the stage timings.
// Returns false on a mismatch.
bool v0_profile_shape(const fa::AttentionShape& s, bool causal, bool check_only, std::ostream* csv,
                      int samples = 30, int warmup = kWarmup)
{
    const size_t n = elements(s);
    std::vector<uint16_t> host(n), plain(n), got(n);
    DeviceBuffer q(n * 2), k(n * 2), v(n * 2), o(n * 2), ws(std::max<size_t>(4, fa::unfused_workspace_bytes(s)));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 11u);
    HIP_OK(hipMemcpy(q.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 22u);
    HIP_OK(hipMemcpy(k.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 33u);
    HIP_OK(hipMemcpy(v.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    float* wsp = static_cast<float*>(ws.ptr);
    hipStream_t stream = nullptr;
    HIP_OK(hipStreamCreate(&stream));
    hipEvent_t ev[6];
    for (auto& e : ev) HIP_OK(hipEventCreate(&e));
    const fa::V0ProfileEvents events{ev[0], ev[1], ev[2], ev[3]};

    HIP_OK(hipMemset(o.ptr, 0xff, n * 2));
    fa::launch_attention_unfused(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal, stream);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipMemcpy(plain.data(), o.ptr, n * 2, hipMemcpyDeviceToHost));
    bool same = true;
    for (const fa::V0ProfileEvents* e : {&events, static_cast<const fa::V0ProfileEvents*>(nullptr)})
    {
        HIP_OK(hipMemset(o.ptr, 0xff, n * 2));
        HIP_OK(fa::launch_attention_unfused_profile(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal, e,
                                                    stream));
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipMemcpy(got.data(), o.ptr, n * 2, hipMemcpyDeviceToHost));
        size_t nan = 0, inf = 0;
        count_nonfinite(got, nan, inf);
        same = same && nan == 0 && inf == 0 && std::memcmp(got.data(), plain.data(), n * 2) == 0;
    }
    std::printf("v0 profile B=%d H=%d N=%d D=%d causal=%d: %s\n", s.batch, s.heads, s.seq_len, s.head_dim,
                causal ? 1 : 0, same ? "PASS (finite, bitwise equal to v0)" : "FAIL");
    if (same && !check_only)
    {
        for (int i = 0; i < warmup; ++i)
        {
            fa::launch_attention_unfused(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal, stream);
            HIP_OK(fa::launch_attention_unfused_profile(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal,
                                                        nullptr, stream));
        }
        HIP_OK(hipGetLastError());
        HIP_OK(hipStreamSynchronize(stream));
        std::vector<double> t[5];
        for (int i = 0; i < samples; ++i)
        {
            // an unmarked v0 launch between its own events, then the instrumented one
            HIP_OK(hipEventRecord(ev[4], stream));
            fa::launch_attention_unfused(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal, stream);
            HIP_OK(hipEventRecord(ev[5], stream));
            HIP_OK(fa::launch_attention_unfused_profile(q.bf16(), k.bf16(), v.bf16(), o.bf16(), wsp, s, causal,
                                                        &events, stream));
            HIP_OK(hipEventSynchronize(ev[3]));
            const std::pair<int, int> spans[5] = {{0, 1}, {1, 2}, {2, 3}, {0, 3}, {4, 5}};
            for (int m = 0; m < 5; ++m)
            {
                float ms = 0.0f;
                HIP_OK(hipEventElapsedTime(&ms, ev[spans[m].first], ev[spans[m].second]));
                t[m].push_back(ms);
            }
        }
        const char* labels[5] = {"QK", "softmax", "PV", "instrumented_pipeline", "original_v0_e2e"};
        const double pipeline = quantile_of(t[3], 0.5);
        char tag[64];
        std::snprintf(tag, sizeof(tag), "b%dh%dn%dd%d_%s", s.batch, s.heads, s.seq_len, s.head_dim,
                      causal ? "causal" : "dense");
        std::printf("  %-22s %10s %10s %10s %10s %7s\n", "metric", "median_ms", "q1_ms", "q3_ms", "iqr_ms", "share");
        for (int m = 0; m < 5; ++m)
        {
            const double med = quantile_of(t[m], 0.5), q1 = quantile_of(t[m], 0.25), q3 = quantile_of(t[m], 0.75);
            std::printf("  %-22s %10.6f %10.6f %10.6f %10.6f", labels[m], med, q1, q3, q3 - q1);
            *csv << tag << ',' << s.batch << ',' << s.heads << ',' << s.seq_len << ',' << s.head_dim << ','
                 << (causal ? 1 : 0) << ',' << labels[m] << ',' << med << ',' << q1 << ',' << q3 << ',' << q3 - q1
                 << ',';
            if (m < 4)
            {
                std::printf(" %7.4f", med / pipeline);
                *csv << med / pipeline;
            }
            std::printf("\n");
            *csv << '\n';
        }
    }
    for (auto& e : ev) HIP_OK(hipEventDestroy(e));
    HIP_OK(hipStreamDestroy(stream));
    return same;
}

// The profiler mode: `iterations` instrumented v0 launches with no events,
// no validation and no warmup, so a profiler sees exactly those kernels.
bool v0_profile_launches(const fa::AttentionShape& s, bool causal, int iterations)
{
    const size_t n = elements(s);
    std::vector<uint16_t> host(n);
    DeviceBuffer q(n * 2), k(n * 2), v(n * 2), o(n * 2), ws(std::max<size_t>(4, fa::unfused_workspace_bytes(s)));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 11u);
    HIP_OK(hipMemcpy(q.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 22u);
    HIP_OK(hipMemcpy(k.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    fa_oracle_fill_normal_mt19937(host.data(), static_cast<int64_t>(n), 33u);
    HIP_OK(hipMemcpy(v.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
    for (int i = 0; i < iterations; ++i)
        HIP_OK(fa::launch_attention_unfused_profile(q.bf16(), k.bf16(), v.bf16(), o.bf16(),
                                                    static_cast<float*>(ws.ptr), s, causal, nullptr, nullptr));
    HIP_OK(hipDeviceSynchronize());
    std::vector<uint16_t> got(n);
    HIP_OK(hipMemcpy(got.data(), o.ptr, n * 2, hipMemcpyDeviceToHost));
    size_t nan = 0, inf = 0;
    count_nonfinite(got, nan, inf);
    std::printf("v0 profiler launches B=%d H=%d N=%d D=%d causal=%d: %d iteration(s), output %s\n", s.batch, s.heads,
                s.seq_len, s.head_dim, causal ? 1 : 0, iterations, nan == 0 && inf == 0 ? "finite" : "NOT finite");
    return nan == 0 && inf == 0;
}

}  // namespace

namespace {

// The v0 workspace of one grid case (benchmarks/bench_flash_attention.cu:614-629):
// an allocation that fails for lack of device memory is not an error. It
// prints a note, clears HIP's error state, and returns nullptr, so v0 is
// skipped for that case while the run goes on; any other failure stops the
// run. A request above `cap` bytes (--workspace-cap) takes the same path
// without asking the device, so it can be exercised on purpose.
void* allocate_workspace(size_t bytes, size_t cap, const fa::AttentionShape& s)
{
    void* ws = nullptr;
    const hipError_t status = bytes > cap ? hipErrorOutOfMemory : hipMalloc(&ws, bytes);
    if (status == hipErrorOutOfMemory)
    {
        if (bytes <= cap)
        {
            const hipError_t last = hipGetLastError();
            if (last != hipErrorOutOfMemory) HIP_OK(last);
        }
        std::fprintf(stderr, "V0 workspace allocation failed: B=%d H=%d N=%d D=%d, %.1f MiB.\n", s.batch, s.heads,
                     s.seq_len, s.head_dim, bytes / (1024.0 * 1024.0));
        return nullptr;
    }
    HIP_OK(status);
    return ws;
}

// Why a table entry does not run for a grid case, or nullptr when it runs
// (benchmarks/bench_flash_attention.cu:655-656).
const char* skip_reason(bool supported, bool needs_workspace, bool have_workspace)
{
    if (!supported) return "unsupported";
    if (needs_workspace && !have_workspace) return "workspace_allocation_failed";
    return nullptr;
}

// The summary.csv row of a skipped entry: status = the reason, no timing
// columns, the traffic model and the workspace size (:657-666).
void write_skip_row(std::ostream& csv, const char* name, const fa::AttentionShape& s, bool causal, const char* reason,
                    double model_gb, size_t workspace_bytes)
{
    key(csv, name, s, causal);
    csv << ',' << reason << ",0,0,,,,,,,," << model_gb << ',' << workspace_bytes << ",,\n";
}

}  // namespace

#ifndef FA_HARNESS_NO_MAIN
int main(int argc, char** argv)
{
    bool quick = false, accuracy_only = false, v0_profile = false, check_only = false, profiler = false;
    size_t workspace_cap = SIZE_MAX;  // --workspace-cap=BYTES
    std::filesystem::path out_dir = "results/raw/flash_attention";
    std::vector<int> numbers;  // --v0-profile shape: B H N D causal [samples [warmup] | iterations]
    auto usage = [&](int status) {
        std::printf("usage: %s [--quick | --accuracy-only] [--workspace-cap=BYTES] [output_directory]\n"
                    "       %s --v0-profile [--check] [output_directory]\n"
                    "       %s --v0-profile B H N D causal [samples [warmup]] [output_directory]\n"
                    "       %s --v0-profile --profiler B H N D causal [iterations]\n",
                    argv[0], argv[0], argv[0], argv[0]);
        return status;
    };
    for (int a = 1; a < argc; ++a)
    {
        const std::string arg = argv[a];
        char* end = nullptr;
        const long value = std::strtol(arg.c_str(), &end, 10);
        if (arg == "--quick") quick = true;
        else if (arg == "--accuracy-only") accuracy_only = true;
        else if (arg == "--v0-profile") v0_profile = true;
        else if (arg == "--check") check_only = true;
        else if (arg == "--profiler") profiler = true;
        else if (arg.rfind("--workspace-cap=", 0) == 0)
        {
            const std::string num = arg.substr(16);
            char* cap_end = nullptr;
            const unsigned long long cap = std::strtoull(num.c_str(), &cap_end, 10);
            if (num.empty() || *cap_end != '\0') return usage(2);
            workspace_cap = static_cast<size_t>(cap);
        }
        else if (arg == "--help" || arg == "-h") return usage(0);
        else if (arg.rfind("--", 0) == 0) return usage(2);
        else if (v0_profile && !arg.empty() && *end == '\0' && value >= 0 && value <= 1 << 30)
            numbers.push_back(static_cast<int>(value));
        else out_dir = arg;
    }
    const size_t max_numbers = profiler ? 6 : 7;
    if (!numbers.empty() && (numbers.size() < 5 || numbers.size() > max_numbers || check_only)) return usage(2);
    if (profiler && numbers.empty()) return usage(2);
    if (!numbers.empty() && (numbers[0] < 1 || numbers[1] < 1 || numbers[2] < 1 || numbers[3] < 1 || numbers[4] > 1))
        return usage(2);
    std::error_code ec;
    std::filesystem::create_directories(out_dir, ec);
    if (ec)
    {
        std::fprintf(stderr, "cannot create %s: %s\n", out_dir.string().c_str(), ec.message().c_str());
        return 2;
    }
    if (v0_profile)
    {
        bool ok = true;
        std::ofstream stage_csv;
        if (!check_only && !profiler)
            stage_csv = open_csv(out_dir / "v0_stage_timing.csv",
                                 "shape,batch,heads,seq_len,head_dim,causal,metric,median_ms,q1_ms,q3_ms,iqr_ms,"
                                 "share_of_pipeline");
        if (!numbers.empty())
        {
            const fa::AttentionShape shape{numbers[0], numbers[1], numbers[2], numbers[3]};
            const bool causal = numbers[4] != 0;
            if (profiler) ok = v0_profile_launches(shape, causal, numbers.size() > 5 ? std::max(1, numbers[5]) : 1);
            else
                ok = v0_profile_shape(shape, causal, false, &stage_csv, numbers.size() > 5 ? std::max(1, numbers[5]) : 30,
                                      numbers.size() > 6 ? numbers[6] : kWarmup);
        }
        else if (check_only)
        {
            for (int n : {1, 17, 256})
                for (int d : {64, 128})
                    for (bool causal : {false, true}) ok = v0_profile_shape({1, 2, n, d}, causal, true, nullptr) && ok;
        }
        else
        {
            // the reference's two profiling shapes (results/raw/v0_stage_timing.csv)
            ok = v0_profile_shape({2, 8, 2048, 64}, false, false, &stage_csv) && ok;
            ok = v0_profile_shape({1, 8, 2048, 128}, false, false, &stage_csv) && ok;
        }
        return ok ? 0 : 1;
    }
    auto raw_csv = open_csv(out_dir / "raw_timings.csv", "kernel,batch,heads,seq_len,head_dim,causal,iteration,elapsed_ms");
    auto summary_csv = open_csv(out_dir / "summary.csv",
                                "kernel,batch,heads,seq_len,head_dim,causal,status,warmup_iters,timed_iters,"
                                "median_ms,q1_ms,q3_ms,iqr_ms,baseline_median_ms,speedup_vs_v0,"
                                "tflops,algorithmic_hbm_gb,v0_workspace_bytes,output_nan,output_inf");
    auto accuracy_csv = open_csv(out_dir / "accuracy.csv",
                                 "kernel,batch,heads,seq_len,head_dim,causal,vs_double,row_scaled_error,"
                                 "max_abs_error,row_scale_ulp,output_nan,output_inf,reference_nan,reference_inf,"
                                 "passed,abs_gate");

    hipDeviceProp_t props{};
    HIP_OK(hipGetDeviceProperties(&props, 0));
    std::printf("device: %s (%s, %d CUs)\n", props.name, props.gcnArchName, props.multiProcessorCount);
    std::printf("timing: %d warmups, %d individually event-timed launches; median and IQR\n\n", kWarmup, kTimed);

    std::printf("fused kernel resources:\n  %-14s %8s %6s %8s %8s %12s %6s %7s %10s\n", "kernel", "head_dim", "block",
                "tile_kv", "q_rows", "shared/block", "regs", "local", "blocks/CU");
    for (int d : {64, 128})
        for (const auto& [name, info] : {std::pair{"v3_tensorcore", fa::query_tensorcore_v3(d)},
                                         std::pair{"v3b_tensorcore", fa::query_tensorcore_v3b(d)}})
            std::printf("  %-14s %8d %6d %8d %8d %11dB %6d %6dB %10d\n", name, d, info.block_size, info.tile_kv,
                        info.rows_per_block, info.shared_bytes_per_block, info.registers_per_thread,
                        info.local_bytes_per_thread, info.max_blocks_per_sm);
    // Every workgroup configuration of the MFMA kernel (v3 picks one per
    // shape; the "v3 rows" column of the grid below says which), with the
    // AGPRs of the compiler's resource report.
    std::printf("\nMFMA kernel configurations (fa_query_fused_groups):\n  %8s %9s %8s %6s %6s %6s %6s %12s %10s\n",
                "q_rows", "kv_groups", "head_dim", "waves", "block", "VGPRs", "AGPRs", "shared/block", "blocks/CU");
    for (const auto& [rows, groups] : {std::pair{64, 2}, std::pair{64, 4}, std::pair{128, 2}, std::pair{128, 4}, std::pair{256, 1}})
        for (int d : {64, 128})
        {
            fa_tiling_info info{};
            if (fa_query_fused_groups(d, rows, groups, &info) != 0) return 2;
            if (!info.supported)
            {
                std::printf("  %8d %9d %8d  (no configuration)\n", rows, groups, d);
                continue;
            }
            std::printf("  %8d %9d %8d %6d %6d %6d %6d %11dB %10d\n", rows, groups, d, info.waves_per_block,
                        info.block_size, info.registers_per_thread, info.agprs_per_thread, info.shared_bytes_per_block,
                        info.max_blocks_per_sm);
        }
    // The kernel v3 itself launches at BASELINE's four metric shapes: its
    // configuration and the instantiation for the mask (dense and causal
    // builds of a configuration differ in registers, spills and occupancy).
    std::printf("\nv3 at the metric shapes (fa_tensorcore_v3_config, query_tensorcore_v3(shape, causal)):\n"
                "  %-18s %6s %8s %9s %6s %6s %6s %12s %10s\n",
                "shape", "mask", "q_rows", "kv_groups", "VGPRs", "AGPRs", "local", "shared/block", "blocks/CU");
    for (int d : {64, 128})
        for (bool causal : {false, true})
        {
            const fa::AttentionShape s{2, 8, 2048, d};
            int rows = 0, groups = 0;
            if (fa_tensorcore_v3_config(s.batch, s.heads, s.seq_len, d, causal ? 1 : 0, &rows, &groups) != 0) return 2;
            fa_tiling_info info{};
            if (fa_query_tensorcore_v3_shape(s.batch, s.heads, s.seq_len, d, causal ? 1 : 0, &info) != 0) return 2;
            const fa::FusedTilingInfo cpp = fa::query_tensorcore_v3(s, causal);
            if (cpp.registers_per_thread != info.registers_per_thread || cpp.rows_per_block != info.rows_per_block)
                return 2;
            char name[32];
            std::snprintf(name, sizeof(name), "(2,8,2048,%d)", d);
            std::printf("  %-18s %6s %8d %9d %6d %6d %5dB %11dB %10d\n", name, causal ? "causal" : "dense", rows,
                        groups, info.registers_per_thread, info.agprs_per_thread, info.local_bytes_per_thread,
                        info.shared_bytes_per_block, info.max_blocks_per_sm);
        }
    std::printf("\n");

    const std::vector<Entry> table = entries();
    bool all_ok = true;

    // Accuracy suite: the reference's shape and inputs.
    std::printf("accuracy (1,2,256), reference inputs:\n  %-16s %5s %6s %11s %11s %11s %7s %8s %6s\n", "kernel", "D",
                "causal", "vs_double", "row_scaled", "max_abs", "ulp", "abs_gate", "status");
    for (int d : {64, 128})
        for (bool causal : {false, true})
        {
            const fa::AttentionShape s{1, 2, 256, d};
            const size_t n = elements(s);
            std::vector<uint16_t> hq(n), hk(n), hv(n), ho(n);
            fa_oracle_fill_normal_mt19937(hq.data(), static_cast<int64_t>(n), 11u);
            fa_oracle_fill_normal_mt19937(hk.data(), static_cast<int64_t>(n), 22u);
            fa_oracle_fill_normal_mt19937(hv.data(), static_cast<int64_t>(n), 33u);
            std::vector<double> ref(n);
            if (fa_oracle_attention(hq.data(), hk.data(), hv.data(), ref.data(), s.batch, s.heads, s.seq_len, d,
                                    causal ? 1 : 0, nullptr, 0, 0) != 0)
                return 2;
            DeviceBuffer q(n * 2), k(n * 2), v(n * 2), o(n * 2), ws(fa::unfused_workspace_bytes(s));
            HIP_OK(hipMemcpy(q.ptr, hq.data(), n * 2, hipMemcpyHostToDevice));
            HIP_OK(hipMemcpy(k.ptr, hk.data(), n * 2, hipMemcpyHostToDevice));
            HIP_OK(hipMemcpy(v.ptr, hv.data(), n * 2, hipMemcpyHostToDevice));
            const Problem p{q.bf16(), k.bf16(), v.bf16(), o.bf16(), static_cast<float*>(ws.ptr), s, causal};
            for (const Entry& e : table)
            {
                if (!e.supported(d)) continue;
                HIP_OK(hipMemset(o.ptr, 0xff, n * 2));  // unwritten outputs read as NaN
                e.launch(p);
                HIP_OK(hipGetLastError());
                HIP_OK(hipDeviceSynchronize());
                HIP_OK(hipMemcpy(ho.data(), o.ptr, n * 2, hipMemcpyDeviceToHost));
                fa_oracle_accuracy acc{};
                fa_oracle_compare(ho.data(), ref.data(), static_cast<int64_t>(n / d), d, &acc);
                const bool ok = acc.passed_ulp && acc.passed_abs;
                all_ok = all_ok && ok;
                std::printf("  %-16s %5d %6s %11.4e %11.4e %11.4e %7.2f %8.3f %6s\n", e.name, d, causal ? "yes" : "no",
                            acc.vs_double, acc.row_scaled, acc.max_abs, acc.ulp, acc.abs_gate, ok ? "PASS" : "FAIL");
                key(accuracy_csv, e.name, s, causal);
                accuracy_csv << ',' << acc.vs_double << ',' << acc.row_scaled << ',' << acc.max_abs << ',' << acc.ulp
                             << ',' << acc.output_nan << ',' << acc.output_inf << ',' << acc.reference_nan << ','
                             << acc.reference_inf << ',' << (ok ? 1 : 0) << ',' << acc.abs_gate << '\n';
            }
        }
    accuracy_csv.flush();
    std::printf("\n");
    if (accuracy_only)
    {
        std::printf("%s\n", all_ok ? "accuracy suite passed" : "accuracy suite FAILED");
        return all_ok ? 0 : 1;
    }

    // Timed grid.
    std::vector<int> batches = {1, 2, 4}, lengths = {512, 1024, 2048, 4096, 8192};
    if (quick)
    {
        batches = {1};
        lengths = {512, 2048};
    }
    size_t skipped = 0;
    for (int b : batches)
        for (int nlen : lengths)
            for (int d : {64, 128})
                for (bool causal : {false, true})
                {
                    const fa::AttentionShape s{b, 8, nlen, d};
                    const size_t n = elements(s);
                    std::vector<uint16_t> host(n);
                    DeviceBuffer q(n * 2), k(n * 2), v(n * 2), o(n * 2);
                    fa_oracle_fill_uniform(host.data(), static_cast<int64_t>(n), grid_seed(11, s));
                    HIP_OK(hipMemcpy(q.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
                    fa_oracle_fill_uniform(host.data(), static_cast<int64_t>(n), grid_seed(22, s));
                    HIP_OK(hipMemcpy(k.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
                    fa_oracle_fill_uniform(host.data(), static_cast<int64_t>(n), grid_seed(33, s));
                    HIP_OK(hipMemcpy(v.ptr, host.data(), n * 2, hipMemcpyHostToDevice));
                    const size_t ws_bytes = fa::unfused_workspace_bytes(s);
                    void* ws = allocate_workspace(ws_bytes, workspace_cap, s);
                    const bool have_ws = ws != nullptr;
                    const Problem p{q.bf16(), k.bf16(), v.bf16(), o.bf16(), static_cast<float*>(ws), s, causal};
                    // 4*B*H*N^2*D, halved for causal (BASELINE's convention)
                    const double flops = 4.0 * b * s.heads * static_cast<double>(nlen) * nlen * d * (causal ? 0.5 : 1.0);
                    int cfg_rows = 0, cfg_groups = 0;
                    (void)fa_tensorcore_v3_config(b, 8, nlen, d, causal ? 1 : 0, &cfg_rows, &cfg_groups);
                    std::printf("B=%d H=8 N=%d D=%d %s (v3: %d rows per workgroup, %d KV groups)\n"
                                "  %-16s %10s %10s %9s %9s %9s\n",
                                b, nlen, d, causal ? "causal" : "dense", cfg_rows, cfg_groups, "kernel", "median ms",
                                "IQR ms", "TFLOPS", "HBM GB", "speedup");
                    double baseline_ms = 0.0;
                    for (const Entry& e : table)
                    {
                        const double gb = e.hbm_bytes(s, causal) / 1e9;
                        const char* skip = skip_reason(e.supported(d), e.needs_workspace, have_ws);
                        if (skip)
                        {
                            ++skipped;
                            std::printf("  %-16s SKIP (%s)\n", e.name, skip);
                            write_skip_row(summary_csv, e.name, s, causal, skip, gb, ws_bytes);
                            continue;
                        }
                        HIP_OK(hipMemset(o.ptr, 0xff, n * 2));
                        const Summary t = time_entry(e, p);
                        std::vector<uint16_t> out(n);
                        HIP_OK(hipMemcpy(out.data(), o.ptr, n * 2, hipMemcpyDeviceToHost));
                        size_t nan = 0, inf = 0;
                        count_nonfinite(out, nan, inf);
                        const bool finite = nan == 0 && inf == 0;
                        all_ok = all_ok && finite;
                        if (std::strcmp(e.name, "v0_unfused") == 0 && finite) baseline_ms = t.median;
                        const double tflops = flops / (t.median * 1e-3) / 1e12;
                        const bool have_speedup = baseline_ms > 0.0 && finite;
                        std::printf("  %-16s %10.4f %10.4f %9.1f %9.3f", e.name, t.median, t.q3 - t.q1, tflops, gb);
                        if (have_speedup) std::printf(" %8.2fx", baseline_ms / t.median);
                        std::printf("%s\n", finite ? "" : "  NONFINITE");
                        for (size_t it = 0; it < t.raw.size(); ++it)
                        {
                            key(raw_csv, e.name, s, causal);
                            raw_csv << ',' << it + 1 << ',' << t.raw[it] << '\n';
                        }
                        key(summary_csv, e.name, s, causal);
                        summary_csv << ',' << (finite ? "ok" : "nonfinite_output") << ',' << kWarmup << ','
                                    << t.raw.size() << ',' << t.median << ',' << t.q1 << ',' << t.q3 << ','
                                    << t.q3 - t.q1 << ',';
                        if (baseline_ms > 0.0) summary_csv << baseline_ms;
                        summary_csv << ',';
                        if (have_speedup) summary_csv << baseline_ms / t.median;
                        summary_csv << ',' << tflops << ',' << gb << ',' << ws_bytes << ',' << nan << ',' << inf << '\n';
                    }
                    if (ws) HIP_OK(hipFree(ws));
                    raw_csv.flush();
                    summary_csv.flush();
                }
    std::printf("\n%s; %zu kernel/shape runs skipped; CSV files in %s\n",
                all_ok ? "all accuracy rows passed and all timed outputs are finite" : "FAILED", skipped,
                out_dir.string().c_str());
    return all_ok ? 0 : 1;
}
#endif  // FA_HARNESS_NO_MAIN
