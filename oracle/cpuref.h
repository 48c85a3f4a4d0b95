/* The oracle: a plain-C restatement of the reference's CPU forward (CpuRef F32 and F64), used ONLY as the checker by
 * the tests, by the smoke check and by the bench's CPU-baseline leg. It is test infrastructure, never the product:
 * nothing in rosylnalive_amd/ links or calls it.
 *
 * Every function follows src/Lrm.Tensor.CpuReference/{Rows,CpuRef,Rope,CpuExec}.fs and
 * tests/Lrm.Tensor.Tests/TinyModel.fs of the reference:
 *   - reductions are sequential in increasing index order from +0 (Rows.fs:28-45);
 *   - products inside a reduction are fused: acc = fma(x, y, acc), one rounding (Rows.fs:33,43);
 *   - element-wise formulas round after every operation in the order written (cpu-reference.md rule 4);
 *   - division and sqrt are IEEE; exp/log come from the C runtime (the reference takes them from .NET, so their
 *     last bit is not pinned by anything committed in the reference: see the parity notes in the tests);
 *   - work is split over threads only across independent outputs (CpuExec.fs:35-49), so the bits do not depend on
 *     the thread count.
 * Every entry point returns 0 on success and a negative code on an argument error (where the reference raises
 * ArgumentException / ArgumentOutOfRangeException); orc_last_error() returns the message.
 */
#ifndef LRM_ORACLE_CPUREF_H
#define LRM_ORACLE_CPUREF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *orc_last_error(void);
void orc_set_threads(int n);
int orc_get_threads(void);

/* bf16 (src/Lrm.Core/Numerics.fs:24-45). */
float orc_bf16_widen(uint16_t bits);
uint16_t orc_bf16_narrow_rne(float x);

/* Correctly rounded float64 cos/sin of a float32 (Rope.fs:146-161) and the T_spec table (Rope.fs:218-251). */
int orc_cos_sin_exact(float x, double *c, double *s);
int orc_rope_table(const uint32_t *inv_freq_bits, int half, int max_pos, float *cos_out, float *sin_out);

/* head_dim ** -0.5 in float64, rounded once (CpuRef.fs:56-60). */
float orc_attention_scale_f32(int head_dim);
double orc_attention_scale_f64(int head_dim);

/* Tensor ops, one per mode (CpuRef.fs). Shapes are passed explicitly; tensors are row-major. */
#define ORC_DECLARE_OPS(T, S)                                                                                        \
    int orc_embed_##S(const uint16_t *table, int vocab, int cols, const int32_t *ids, int rows, T *y);               \
    int orc_embed_gather_##S(const uint16_t *table, int vocab, int cols, const uint32_t *ids, int rows, T *y);       \
    int orc_rmsnorm_##S(const T *x, int64_t elems, const uint16_t *w, int width, T eps, T *y);                       \
    int orc_matmul_bf16w_##S(const T *x, int m, int k, const uint16_t *w, int n, T *y);                             \
    int orc_rope_apply_##S(const float *cos_t, const float *sin_t, int max_pos, int half, const T *x, int rows,      \
                           int heads, int pos0, T *y);                                                               \
    int orc_attention_##S(const T *q, int rows, const T *k_cache, const T *v_cache, int cache_rows, int q_heads,     \
                          int kv_heads, int head_dim, int past, T scale, T *y);                                      \
    int orc_silu_mul_##S(const T *gate, const T *up, int64_t n, T *y);                                               \
    int orc_add_##S(const T *a, const T *b, int64_t n, T *y);                                                        \
    int orc_copy_rows_##S(const T *src, int src_rows, int src_row0, T *dst, int dst_rows, int dst_row0, int rows,     \
                          int cols);                                                                                 \
    int orc_argmax_rows_##S(const T *x, int rows, int cols, uint32_t *y);                                            \
    int orc_softmax_rows_##S(const T *x, int rows, int cols, T *y);                                                  \
    int orc_logsumexp_rows_##S(const T *x, int rows, int cols, T *y);                                                \
    int orc_kl_rows_##S(const T *p, const T *q, int rows, int cols, T *y);

ORC_DECLARE_OPS(float, f32)
ORC_DECLARE_OPS(double, f64)

/* The Qwen3 decoder forward composed as tests/Lrm.Tensor.Tests/TinyModel.fs:144-204 does.
 * Weights: w[0] = model.embed_tokens.weight [vocab, hidden] (also the tied lm_head), w[1] = model.norm.weight, then
 * per layer i, base 2 + 11 * i: input_layernorm, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm,
 * post_attention_layernorm, gate_proj, up_proj, down_proj (all bf16, PyTorch Linear layout [out, in]).
 * Caches: per layer [max_pos, kv_heads * head_dim] in the mode's dtype, layer i at k_cache + i * max_pos * kv_cols.
 * taps (nullable): 18 * layers + 3 output pointers in ActivationNames order (src/Lrm.Tensor/Goldens.fs:288-320);
 * each non-null pointer receives that tap [T, width]. */
typedef struct orc_qwen_config {
    int layers;
    int hidden;
    int heads;
    int kv_heads;
    int head_dim;
    int intermediate;
    int vocab;
    int max_pos;
    double eps;
} orc_qwen_config;

int orc_qwen_forward_f32(const orc_qwen_config *cfg, const uint16_t *const *w, const float *cos_t, const float *sin_t,
                         float *k_cache, float *v_cache, int pos0, const int32_t *ids, int t, float *logits,
                         float *const *taps);
int orc_qwen_forward_f64(const orc_qwen_config *cfg, const uint16_t *const *w, const float *cos_t, const float *sin_t,
                         double *k_cache, double *v_cache, int pos0, const int32_t *ids, int t, double *logits,
                         double *const *taps);

/* The canonical greedy schedule (TinyModel.fs:219-236): one prefill of the prompt, then steps - 1 single-token
 * decode steps, each choosing the argmax of the last logits row. out_ids receives `steps` ids. */
int orc_qwen_greedy_f32(const orc_qwen_config *cfg, const uint16_t *const *w, const float *cos_t, const float *sin_t,
                        const int32_t *prompt, int prompt_len, int steps, int32_t *out_ids);
int orc_qwen_greedy_f64(const orc_qwen_config *cfg, const uint16_t *const *w, const float *cos_t, const float *sin_t,
                        const int32_t *prompt, int prompt_len, int steps, int32_t *out_ids);

#ifdef __cplusplus
}
#endif

#endif
