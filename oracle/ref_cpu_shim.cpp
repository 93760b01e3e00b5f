// TEST INFRASTRUCTURE ONLY: a C-linkage binding for the reference's own CPU
// kernel, compiled together with the unmodified reference source
// /root/reference/csrc/mla_decode_naive_fp32_cpu.cpp by oracle/Makefile into
// oracle/_ref/libref_mla_cpu.so. It lets the tests load the reference's
// run_mla_decode_cpu (declared at csrc/mla_decode.hpp:3-8) through ctypes to
// pin the oracle restatement; nothing in the product path loads it.

void run_mla_decode_cpu(const float *query, const float *cache, float *out,
                        int num_heads, int head_dim_c, int seq_length);

extern "C" void ref_run_mla_decode_cpu(const float *query, const float *cache,
                                       float *out, int num_heads,
                                       int head_dim_c, int seq_length)
{
    run_mla_decode_cpu(query, cache, out, num_heads, head_dim_c, seq_length);
}
