/* oracle.h — declarations of the CPU oracle (oracle.c).  TEST INFRASTRUCTURE ONLY: for the
 * C/C++ test drivers under tests/; the product never includes this header. */
#ifndef EI_ORACLE_H
#define EI_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
void orc_fill_normal(float* out, size_t n, uint64_t seed, uint64_t offset);
void orc_fill_gamma(float* out, size_t n, uint64_t seed);
void orc_rmsnorm(float* out, const float* x, const float* w, int n, float eps);
/* y[r] = dot(row r of w, x) for `rows` rows of n values in the GGUF layout of `type` (0 F32, 1 F16, 8 Q8_0,
 * 12 Q4_K, 14 Q6_K) */
void orc_matvec(int type, const void* w, const float* x, float* y, long rows, long n);
void orc_rope_inv_freq(double* out, int rope_dim, double base);
void orc_rope(float* v, int pos, int dim, const double* inv_freq);
void orc_rope_table(float* cs, int n_ctx, int rope_dim, double base);
void orc_headnorm_rope(float* buf, int rows, long row_stride, int n_heads, int D, const float* gamma, int pos0,
                       int rope_dim, double base, float eps);
void orc_kv_append(const float* k_src, const float* v_src, long src_stride, int rows, float* kc, float* vc, int kd,
                   int pos0);
void orc_attn_decode(const float* q, const float* kc, const float* vc, float* out, int T, int H, int HKV, int D,
                     float scale, float* scores);
void orc_attn_prefill(const float* q, long q_stride, const float* kc, const float* vc, float* out, int B, int pos0,
                      int H, int HKV, int D, float scale);
void orc_attn_f64(const float* q, const float* kc, const float* vc, double* out, int T, int H, int HKV, int D,
                  double scale);
int orc_threads(void);
void orc_set_threads(int n);
#ifdef __cplusplus
}
#endif
#endif
