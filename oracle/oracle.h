/*
 * CPU parity oracle for the KuiperLLama batch-1 token-generation path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C++, the CPU
 * semantics of the reference's decode step so that the HIP product can be
 * checked against it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference checkout).  Where the reference has no CPU path (INT8 GEMV,
 * per-head q/k RMSNorm) the CUDA semantics are restated and the comment says
 * so.  Reduction order inside Armadillo/OpenBLAS is not reproducible without
 * the library; the oracle fixes its own order (documented per function) and
 * the product is compared against it within the stated tolerances.
 */
#ifndef KUIPER_ORACLE_H_
#define KUIPER_ORACLE_H_
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model families: the reference selects these with compile-time flags
 * (CMakeLists.txt:29-47); the oracle takes them at run time. */
enum or_family { OR_LLAMA2 = 0, OR_LLAMA3 = 1, OR_QWEN2 = 2, OR_QWEN3 = 3 };
/* RoPE styles: interleaved pairs (i, i+1) and rotate-half pairs (j, j+hd/2). */
enum or_rope_style { OR_ROPE_INTERLEAVED = 0, OR_ROPE_HALF = 1 };

void or_set_threads(int n);
int or_get_threads(void);

/* ---- op level ---- */
void or_gemv_f32(const float* x, const float* W, float* y, int rows, int cols, float scale);
void or_gemv_q8(const float* x, const int8_t* q, const float* scales, float* y, int rows, int cols,
                int group_size);
/* The element-by-element loop of or_gemv_q8 (test hook: or_gemv_q8 takes a
 * vector path where group_size and cols are multiples of 8; tests check the
 * two are bitwise equal). */
void or_gemv_q8_scalar(const float* x, const int8_t* q, const float* scales, float* y, int rows,
                       int cols, int group_size);
void or_quantize_q8(const float* w, int64_t n, int group_size, int8_t* q, float* scales);
void or_dequant_q8(const int8_t* q, const float* scales, int64_t n, int group_size, float* out);
void or_rmsnorm(const float* x, const float* w, float* y, int n, float eps);
void or_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n, float eps);
void or_sincos_table(int head_size, int seq_len, float theta, float* sin_cache, float* cos_cache);
void or_rope(int style, int dim, int kv_dim, int head_size, float* q, float* k, int pos,
             const float* sin_cache, const float* cos_cache);
void or_softmax(float* x, int n);
void or_mha(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
            int head_size, float* out, const float* q, float* score, const float* key_cache,
            const float* value_cache);
void or_scale(float scale, float* x, int n);
void or_scale_sum(const float* value, const float* scale, float* out, int pos, int size, int stride);
void or_swiglu(const float* a, const float* b, float* out, int n);
void or_add(const float* a, const float* b, float* out, int n);
int or_embedding(const int32_t* tokens, int n_tokens, const float* table, int vocab, int dim,
                 float* out);
int64_t or_argmax(const float* x, int64_t n);

/* ---- model level ---- */
typedef struct or_model or_model;
/* Parses a reference-format .bin image held in memory (not copied; must
 * outlive the model).  Returns NULL and fills err on a malformed image. */
or_model* or_model_open(const void* image, size_t size, int family, int quant, char* err,
                        int err_len);
void or_model_close(or_model* m);
/* dims: {dim, q_dim, kv_dim, hidden(FFN), layers, heads, kv_heads, vocab, seq_len, head_size} */
void or_model_dims(const or_model* m, int32_t* out10);
/* One reference forward step (embedding of `token` at `pos` + all layers +
 * final norm + classifier).  logits may be NULL. */
int or_model_step(or_model* m, int32_t token, int32_t pos, float* logits);
/* n_tokens prompt tokens at positions pos0 .. pos0+n_tokens-1, equal bit
 * for bit (logits of the last position, cache rows) to or_model_step on each
 * position in turn, but with each weight row applied to many positions while
 * it is cached.  logits (of the last position) may be NULL.  Returns 0, -1 for
 * a token outside the vocabulary, -2 for positions outside the cache. */
int or_model_prompt(or_model* m, const int32_t* tokens, int n_tokens, int32_t pos0, float* logits);
/* demo/main.cpp:5-47 greedy loop: P prompt tokens, then n_new sampled tokens
 * written to out_tokens.  Returns the number of tokens written. */
int or_model_generate(or_model* m, const int32_t* prompt, int P, int n_new, int32_t* out_tokens);
/* Copies one layer's cache row (K or V) for inspection. */
void or_model_kv_row(const or_model* m, int layer, int pos, int which_v, float* out);

#ifdef __cplusplus
}
#endif
#endif
