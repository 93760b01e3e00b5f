/*
 * TEST INFRASTRUCTURE ONLY. This file is the CPU oracle for the MLA decode
 * path; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker or the reported CPU baseline. The
 * product path never calls it.
 *
 * Restatement of the reference's naive fp32 CPU kernel
 * run_mla_decode_cpu (csrc/mla_decode_naive_fp32_cpu.cpp:5-61), step for
 * step, parameterised by the logit divisor and by the number of value
 * columns so that one function covers both
 *   - the reference's own form: divisor sqrt(576), dv = 576
 *     (csrc/mla_decode_naive_fp32_cpu.cpp:24, :50-58), and
 *   - the decode contract: divisor sqrt(192), dv = 512 (mla.py:44-47).
 *
 * Arithmetic follows the reference exactly:
 *   1. tmp[i][j] = sum_k q[i][k] * c[j][k], accumulated in float in k order
 *      (cpu.cpp:16-22), then tmp /= divisor computed in double and stored as
 *      float (cpu.cpp:24: float /= double).
 *   2. row max in float (cpu.cpp:32-38); sum += exp(tmp - max) where the
 *      subtraction is float, exp is the double-precision exp, and the running
 *      sum is a float (cpu.cpp:39-42: unqualified exp with <cmath> resolves to
 *      ::exp(double)); tmp = exp(tmp - max) / sum in double, stored as float
 *      (cpu.cpp:43-46).
 *   3. out[i][j] = sum_k tmp[i][k] * c[k][j], accumulated in float in k order
 *      (cpu.cpp:50-58), for j < dv.
 * The reference allocates tmp with new[] and frees it with delete
 * (cpu.cpp:13, :60); this restatement uses malloc/free.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math, so that
 * the float/double rounding sequence above is what executes).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Returns 0 on success, -1 on bad arguments, -2 on allocation failure. */
int oracle_mla_decode_cpu(const float *query, const float *cache, float *out,
                          int num_heads, int head_dim_c, int seq_length,
                          int dv, double divisor)
{
    if (!query || !cache || !out || num_heads <= 0 || head_dim_c <= 0 ||
        seq_length <= 0 || dv <= 0 || dv > head_dim_c || !(divisor > 0.0))
        return -1;

    float *tmp = (float *)malloc(sizeof(float) * (size_t)num_heads *
                                 (size_t)seq_length);
    if (!tmp)
        return -2;

    for (int i = 0; i < num_heads; ++i) {
        for (int j = 0; j < seq_length; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < head_dim_c; ++k)
                acc += query[(size_t)i * head_dim_c + k] *
                       cache[(size_t)j * head_dim_c + k];
            tmp[(size_t)i * seq_length + j] = (float)((double)acc / divisor);
        }
    }

    for (int i = 0; i < num_heads; ++i) {
        float *row = tmp + (size_t)i * seq_length;
        float mx = row[0];
        for (int j = 0; j < seq_length; ++j)
            if (row[j] > mx)
                mx = row[j];
        float sum = 0.0f;
        for (int j = 0; j < seq_length; ++j)
            sum = (float)((double)sum + exp((double)(float)(row[j] - mx)));
        for (int j = 0; j < seq_length; ++j)
            row[j] = (float)(exp((double)(float)(row[j] - mx)) / (double)sum);
    }

    for (int i = 0; i < num_heads; ++i) {
        const float *row = tmp + (size_t)i * seq_length;
        for (int j = 0; j < dv; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < seq_length; ++k)
                acc += row[k] * cache[(size_t)k * head_dim_c + j];
            out[(size_t)i * dv + j] = acc;
        }
    }

    free(tmp);
    return 0;
}
