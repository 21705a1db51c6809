/*
 * TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.
 *
 * C declarations of the FP64 oracle library (oracle/liboracle.so, built from
 * oracle/oracle.cpp), for C/C++ test harnesses under tests/. Each function is
 * documented at its definition with the reference file:line it restates.
 */
#ifndef FA_ORACLE_H
#define FA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fa_oracle_accuracy {
    double vs_double;
    double row_scaled;
    double max_abs;
    double ulp;
    double abs_gate;
    int64_t output_nan;
    int64_t output_inf;
    int64_t reference_nan;
    int64_t reference_inf;
    int32_t passed_ulp;
    int32_t passed_abs;
} fa_oracle_accuracy;

void fa_oracle_fill_uniform(uint16_t* out, int64_t n, uint64_t seed);
void fa_oracle_fill_normal_mt19937(uint16_t* out, int64_t n, uint32_t seed);
int fa_oracle_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, double* out, int batch, int heads,
                        int seq_len, int head_dim, int causal, const int64_t* rows, int64_t n_rows, int threads);
void fa_oracle_compare(const uint16_t* got, const double* ref, int64_t n_rows, int head_dim,
                       fa_oracle_accuracy* result);
double fa_oracle_quantile_sorted(const double* sorted, int64_t n, double p);

#ifdef __cplusplus
}
#endif

#endif /* FA_ORACLE_H */
