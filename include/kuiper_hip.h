/*
 * kuiper_hip.h -- C ABI of the MI355X (gfx950) backend for KuiperLLama's
 * batch-1 token-generation loop.
 *
 * Conventions
 *  - Plain pointers, sizes and an opaque stream handle (a hipStream_t passed
 *    as void*; NULL means the library's default stream).  No C++ or torch
 *    types cross this boundary.
 *  - Every function returns int: 0 on success, a positive hipError_t value
 *    for a runtime failure, or a negative KL_E* code for a rejected argument.
 *    Nothing throws or aborts.  kl_error_string() names a code.
 *  - All tensor pointers of the op-level entry points are device pointers,
 *    fp32 unless stated, row-major, exactly as the reference kernels take them.
 *  - Launches are asynchronous on the given stream unless stated.
 *
 * Reference interfaces each group replaces are cited as file:line, relative
 * to the KuiperLLama checkout (kuiper/source/op/kernels/kernels_interface.h is
 * abbreviated KI).
 */
#ifndef KUIPER_HIP_H_
#define KUIPER_HIP_H_
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ---- */
#define KL_OK 0
#define KL_EINVAL (-1)    /* bad argument (shape, null pointer, range) */
#define KL_ENOMEM (-2)    /* device allocation failed */
#define KL_EFORMAT (-3)   /* malformed model image */
#define KL_EUNSUPP (-4)   /* combination the backend does not implement */
#define KL_ETOKEN (-5)    /* token id outside [0, vocab) */
#define KL_EWORKSPACE (-6)/* caller workspace too small */
#define KL_EDEVICE (-7)   /* the device step reported an error (barrier timeout, bad state) */

/* Model families (the reference picks them with -DLLAMA3_SUPPORT /
 * -DQWEN2_SUPPORT / -DQWEN3_SUPPORT, CMakeLists.txt:29-47; here at run time). */
#define KL_FAMILY_LLAMA2 0 /* interleaved RoPE, theta 1e4, eps 1e-5 */
#define KL_FAMILY_LLAMA3 1 /* rotate-half RoPE, theta 5e5, eps 1e-5 */
#define KL_FAMILY_QWEN2 2  /* rotate-half, theta 1e6, eps 1e-6, q/k/v bias */
#define KL_FAMILY_QWEN3 3  /* rotate-half, theta 1e6, eps 1e-6, per-head q/k RMSNorm */

/* RoPE pairings: kernels/cpu/rope_kernel.cpp:98-121 (interleaved) and
 * :18-42 / :58-82 (rotate-half). */
#define KL_ROPE_INTERLEAVED 0
#define KL_ROPE_HALF 1

const char* kl_error_string(int code);

/* ---------------------------------------------------------------------------
 * Runtime: device selection, memory, streams, events.
 * Replaces base::CUDADeviceAllocator (include/base/alloc.h:59-66,
 * source/base/alloc_cu.cpp:7-112: allocate/release/memcpy/memset_zero),
 * kernel::CudaConfig (include/base/cuda_config.h:6-13) and the cudaSetDevice /
 * cudaStreamCreate calls of LLama2Model::init (source/model/llama3.cpp:116-123).
 * ------------------------------------------------------------------------- */
int kl_device_count(int* count);
int kl_set_device(int device);
int kl_device_name(int device, char* buf, int buf_len);
int kl_malloc(void** ptr, size_t bytes);
int kl_free(void* ptr);
int kl_host_alloc(void** ptr, size_t bytes); /* pinned host memory */
int kl_host_free(void* ptr);
int kl_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int kl_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int kl_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int kl_memset_zero(void* ptr, size_t bytes, void* stream);
int kl_stream_create(void** stream);
int kl_stream_destroy(void* stream);
int kl_stream_sync(void* stream);
int kl_device_sync(void);
int kl_event_create(void** event);
int kl_event_destroy(void* event);
int kl_event_record(void* event, void* stream);
int kl_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---------------------------------------------------------------------------
 * Op-level kernels.  Each mirrors one reference kernel typedef (KI:6-47) with
 * the Tensor arguments unpacked to device pointers and sizes.
 * ------------------------------------------------------------------------- */

/* MatmulKernel (KI:9-10; cuda/matmul_kernel.cu:89-109, cpu/matmul_kernel.cpp:5-41):
 * y[r] = scale * sum_c W[r*cols + c] * x[c]. */
int kl_gemv_f32(const float* x, const float* W, float* y, int rows, int cols, float scale,
                void* stream);

/* MatmulKernelQuant (KI:12-14; cuda/matmul_kernel.cu:111-134):
 * y[r] = sum_c x[c] * scales[(r*cols + c) / group_size] * float(q[r*cols + c]).
 * q is int8 [rows x cols]; scales fp32 [rows*cols / group_size]. */
int kl_gemv_q8(const float* x, const int8_t* q, const float* scales, float* y, int rows, int cols,
               int group_size, void* stream);

/* Dequantised weights, out[i] = scales[i / group_size] * float(q[i]): the
 * per-element product inside the reference int8 GEMV (cuda/matmul_kernel.cu:73). */
int kl_dequant_q8(const int8_t* q, const float* scales, int64_t n, int group_size, float* out,
                  void* stream);

/* RMSNormKernel (KI:30-31; cpu/rmsnorm_kernel.cpp:4-33, cuda/rmsnorm_kernel.cu:110-136):
 * y = w * (x / sqrt(mean(x^2) + eps)).  eps is a build flag in the reference
 * (1e-5 Llama, 1e-6 Qwen); here an argument.  y may alias x. */
int kl_rmsnorm(const float* x, const float* w, float* y, int n, float eps, void* stream);

/* RMSNormKernelDim (KI:33-34; cuda/rmsnorm_kernel.cu:138-164): the same on each
 * of `rows` rows of length n with one shared weight vector (Qwen3 q/k norm). */
int kl_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n, float eps,
                    void* stream);

/* sin_cos_cache_calc_cpu (cpu/rope_kernel.cpp:4-16, :44-56, :84-96):
 * sin/cos(pos * theta^(-d/hd)) for pos < seq_len, d < head_size, computed on
 * the host with the same float formula as the reference CPU path and copied
 * to the device tables [seq_len x head_size].  Synchronous. */
int kl_sincos_table(int head_size, int seq_len, float theta, float* sin_dev, float* cos_dev);

/* RoPEKernel (KI:36-39; cpu/rope_kernel.cpp:18-121): rotates q [dim] and the
 * first kv_dim entries' pairs of k in place at position pos. */
int kl_rope(int style, int dim, int kv_dim, int head_size, float* q, float* k, int pos,
            const float* sin_cache, const float* cos_cache, void* stream);

/* MHAKernel (KI:22-28; cpu/mha_kernel.cpp:5-61, cuda/mha_kernel.cu:109-127):
 * per head h (kv head h / kv_mul): softmax_t((q_h . K_t) / sqrt(hd)) . V_t over
 * t in [0, pos], caches [layers][seq_len][kv_dim].  The reference's score
 * buffer [head_num x seq_len] floats (llama3.cpp:485-487) serves as the
 * split workspace: kl_mha_workspace_size() bytes, never more than
 * head_num * seq_len * 4 (0 where one workgroup per kv head covers seq_len),
 * needing no initialisation.  Two launches on the stream when the context
 * spans several workgroups (partials, then their merge). */
int kl_mha_workspace_size(int head_num, int kv_mul, int seq_len, int head_size, size_t* bytes);
int kl_mha(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
           int head_size, float* out, const float* q, void* workspace, size_t workspace_bytes,
           const float* key_cache, const float* value_cache, void* stream);

/* No reference counterpart: kl_mha for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same kernels, plan and result as kl_mha; the split partials live in a
 * library-owned device array of kl_mha_noalloc_max_bytes() bytes (1 MiB) per
 * device, held until the process ends.  A shape whose partials need more
 * (kl_mha_workspace_size) returns KL_EWORKSPACE before any launch.  Calls
 * share the device's array: calls that overlap on one device (different
 * streams, or host threads) race and must be serialised by the caller.
 * Allocates nothing. */
size_t kl_mha_noalloc_max_bytes(void);
int kl_mha_noalloc(int pos, int head_num, int layer_index, int seq_len, int kv_dim, int kv_mul,
                   int head_size, float* out, const float* q, const float* key_cache,
                   const float* value_cache, void* stream);

/* ---- Batched prompt prefill (no reference counterpart: the reference runs
 * the prompt token by token, demo/main.cpp:20-22, and MatmulLayer accepts
 * only a 1-D input, op/matmul.cpp:20).  Row-major, fp32, device pointers. ---- */

/* C[M x N] = A[M x K] . W[N x K]^T (+ bias[N]) (+ C when accumulate != 0): the
 * MatmulKernel product (KI:9-10) for M input rows at once, on the matrix cores
 * (v_mfma_f32_32x32x2f32, 64 x 64 workgroup tiles).  lda, ldw, ldc are row strides in floats.  Needs
 * K, lda, ldw multiples of 4, A, W 16-byte aligned and M x lda, N x ldw under 4 GiB
 * (else KL_EUNSUPP). */
int kl_gemm_f32(const float* A, const float* W, float* C, int M, int N, int K, int lda, int ldw,
                int ldc, const float* bias, int accumulate, void* stream);

/* The same product for up to 3 outputs over one A in one launch (the Q, K
 * and V projections): C[i][M x N[i]] (+)= A . W[i]^T (+ bias[i]); bias may be
 * NULL (or hold NULL entries). */
int kl_gemm_f32_grouped(const float* A, int M, int K, int lda, int n_seg, const float* const* W,
                        float* const* C, const float* const* bias, const int* N, const int* ldw,
                        const int* ldc, int accumulate, void* stream);

/* kl_gemm_f32 with K divided among `splits` (1..16) workgroup slices for
 * narrow outputs: partial products go to the caller's workspace
 * (>= splits*M*N floats, else KL_EWORKSPACE) and are summed in slice order
 * before bias and accumulate apply.  No allocation. */
int kl_gemm_f32_splitk(const float* A, const float* W, float* C, int M, int N, int K, int lda,
                       int ldw, int ldc, const float* bias, int accumulate, int splits,
                       void* workspace, size_t workspace_bytes, void* stream);

/* MatmulKernelQuant (KI:12-14; cuda/matmul_kernel.cu:111-134) on M rows at
 * once: C[M x N] (+)= A[M x K] . dequant(q)^T (+ bias), q int8 [N x K] (dense
 * rows) with scales[(n*K + k) / group_size] (group_size a power of two >= 4),
 * K a multiple of 32.  Split-K and its workspace as kl_gemm_f32_splitk
 * (splits = 1 needs none).  Used by the batched prefill of int8 images. */
int kl_gemm_q8(const float* A, const int8_t* q, const float* scales, int group_size, float* C,
               int M, int N, int K, int lda, int ldc, const float* bias, int accumulate, int splits,
               void* workspace, size_t workspace_bytes, void* stream);

/* fp32 -> three bf16 planes for kl_gemm_x6: x = x0 + x1 + x2 with
 * x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1) (round to nearest
 * even), which hold all 24 significand bits of x.  rows x cols floats (row
 * stride ldx) -> `planes` in the tiled plane format: tiles of 16 rows x 32
 * columns in row-tile-major order, each tile the three planes' 16 x 32
 * elements one after another (element (r, k) of plane p at
 * ((r/16)*(cols/32) + k/32)*1536 + 512*p + 32*(r%16) + k%32).  cols a
 * multiple of 32, ldx of 4, x and planes 16-byte aligned; planes holds
 * kl_split_bf16x3_bytes(rows, cols) bytes.  No counterpart in the reference:
 * the operand format of the split-product prefill GEMM below. */
size_t kl_split_bf16x3_bytes(int rows, int cols);
int kl_split_bf16x3(const float* x, int rows, int cols, int ldx, void* planes, void* stream);

/* C[M x N] (+)= A . W^T (+ bias) from the planes of A (M x K) and W (N x K)
 * as kl_split_bf16x3 writes them: the six products Ai Wj^T with i + j <= 2 on
 * the bf16 matrix cores, accumulated in fp32, as accurate as an fp32 GEMM
 * (the terms left out are each below one fp32 rounding of |a w|).  The
 * batched form of MatmulLayer (op/matmul.cpp:20) that the prefill runs for
 * fp32 weights.  K a multiple of 32, planes 16-byte aligned.  With a
 * workspace the launch divides K among up to 8 slices where that fills the
 * device (splits * M * N floats, within workspace_bytes); NULL runs one
 * slice. */
int kl_gemm_x6(const void* a_planes, const void* w_planes, float* C, int M, int N, int K, int ldc,
               const float* bias, int accumulate, void* workspace, size_t workspace_bytes,
               void* stream);
/* kl_gemm_x6 told how many of W's planes carry bits (no reference
 * counterpart: a fast path for weights exported from bf16 checkpoints).
 * w_planes_used 1: W's planes 1 and 2 are all zero (every weight a bf16 value,
 * see kl_x6_weight_planes), so only the three products Ai W0^T are formed --
 * the same values as kl_gemm_x6, whose other three terms are then exact
 * zeros; on W with nonzero planes 1 or 2 it drops them.  3: kl_gemm_x6.  Else
 * KL_EINVAL. */
int kl_gemm_x6w(const void* a_planes, const void* w_planes, int w_planes_used, float* C, int M, int N,
                int K, int ldc, const float* bias, int accumulate, void* workspace,
                size_t workspace_bytes, void* stream);
/* *planes_used = 1 if planes 1 and 2 of W (N x K, kl_split_bf16x3's format)
 * are all zero, else 3; synchronous on stream (allocates one word). */
int kl_x6_weight_planes(const void* w_planes, int N, int K, int* planes_used, void* stream);

/* MatmulKernelQuant (KI:12-14; cuda/matmul_kernel.cu:111-134) for prompts of
 * at most 32 rows, bound by the int8 weight bytes: the weights prepacked once
 * (kl_q8s_pack: q int8 [N x K] dense rows, scales[(n*K + k) / group_size],
 * group_size 32 or 64 dividing K, into kl_q8s_packed_bytes bytes,
 * 16-byte aligned), then C[M x N] (+)= A . dequant(q)^T (+ bias) as sum over
 * groups of scale * (sum of a*q over the group): A as three bf16 planes and q
 * exactly in bf16, three products per multiply-add on the bf16 matrix cores,
 * fp32 accumulation (as accurate as the fp32 GEMM).  The workspace holds A's
 * planes (K * 192 bytes, else KL_EWORKSPACE) and, beyond them (at the next
 * 256-byte boundary), split-K partials where they fit (splits * M * N
 * floats); a split holds at most 832 columns of K, so K > 832 needs room for
 * ceil(K / 832) splits or more (else KL_EWORKSPACE).  M <= 32.  No
 * counterpart of the packed format in the reference. */
size_t kl_q8s_packed_bytes(int N, int K, int group_size);
int kl_q8s_pack(const int8_t* q, const float* scales, int N, int K, int group_size, void* packed,
                void* stream);
int kl_gemm_q8s(const float* A, int M, int K, int lda, const void* packed, int N, int group_size,
                float* C, int ldc, const float* bias, int accumulate, void* workspace,
                size_t workspace_bytes, void* stream);

/* RoPEKernel (KI:36-39) on n_pos rows: row r of q (stride ldq) and of k
 * (stride ldk) rotated at position pos0 + r. */
int kl_rope_rows(int style, int dim, int kv_dim, int head_size, float* q, int ldq, float* k,
                 int ldk, int pos0, int n_pos, const float* sin_cache, const float* cos_cache,
                 void* stream);

/* Qwen3's per-head q/k RMSNorm (model/qwen3.cpp:485-500; RMSNormKernelDim
 * semantics, y = w * (x / sqrt(mean(x^2) + eps))) followed by RoPEKernel on
 * n_pos prefill rows in one pass (no reference counterpart for the fusion:
 * the reference applies the two per token).  Row r of q (q_heads heads,
 * stride ldq) and of k (kv_heads heads, stride ldk) at position pos0 + r;
 * every k head is rotated.  head_size 64 or 128, and q, k, the norm weights
 * and the sin/cos tables 16-byte aligned with ldq, ldk multiples of 4 (else
 * KL_EUNSUPP); the same values as kl_rmsnorm_rows then kl_rope_rows up to
 * float rounding. */
int kl_qk_norm_rope_rows(int style, int head_size, int q_heads, int kv_heads, float* q, int ldq,
                         float* k, int ldk, const float* q_norm, const float* k_norm, float eps,
                         int pos0, int n_pos, const float* sin_cache, const float* cos_cache,
                         void* stream);

/* MHAKernel (KI:22-28) for query positions pos0 .. pos0+n_pos-1 at once:
 * row r of q (stride ldq, head_num*head_size floats) attends key/value rows
 * 0 .. pos0+r of one layer's caches ([seq_len][kv_dim]), causal; out row r
 * (stride ldo).  head_size 32, 64, 128 or 256 (else KL_EUNSUPP).  Head sizes
 * 64 and 128 run on the matrix cores: 128 with the products as split bf16
 * terms (x = x0 + x1 + x2, six partial products, as accurate as fp32
 * products; KL_PREFILL_ATTN=f32 in the environment selects the fp32 products),
 * 64 with fp32 products. */
int kl_attn_prefill(int pos0, int n_pos, int head_num, int kv_mul, int head_size, const float* q,
                    int ldq, const float* key_cache, const float* value_cache, int kv_dim,
                    float* out, int ldo, void* stream);
/* kl_attn_prefill with a workspace (no reference counterpart for the split
 * itself; same MHAKernel semantics).  Head sizes 64 and 128: where the causal
 * (64-row block, head) segments are unequal or fewer than the CUs, one
 * workgroup per CU takes an equal share of the (row block, 64-key block)
 * units; a segment cut between workgroups leaves partial (max, sum, output)
 * rows in the workspace, and a merge pass combines them in key order.
 * workspace: kl_attn_prefill_workspace_size bytes, 16-byte aligned, no
 * initialisation needed (launches sharing one workspace must not overlap);
 * KL_EWORKSPACE if smaller.  0 bytes for head size 32, which runs
 * kl_attn_prefill, as does a launch that the split would not shorten. */
int kl_attn_prefill_workspace_size(int n_pos, int head_num, int head_size, size_t* bytes);
int kl_attn_prefill_ws(int pos0, int n_pos, int head_num, int kv_mul, int head_size, const float* q,
                       int ldq, const float* key_cache, const float* value_cache, int kv_dim,
                       float* out, int ldo, void* workspace, size_t workspace_bytes, void* stream);

/* SwigluKernel (KI:19-20; cpu/swiglu_kernel.cpp:3-23): out = a*sigmoid(a)*b. */
int kl_swiglu(const float* a, const float* b, float* out, int n, void* stream);

/* AddKernel (KI:6-7; cpu/add_kernel.cpp:5-19): out = a + b. */
int kl_add(const float* a, const float* b, float* out, int n, void* stream);

/* ScaleKernel (KI:41; cpu/scale_kernel.cpp:3-9): x = x * scale in place. */
int kl_scale(float scale, float* x, int n, void* stream);

/* SoftmaxInplaceKernel (KI:43; cpu/softmax_kernel.cpp:4-16): x = exp(x - max x)
 * / sum, in place over one vector of n floats (one workgroup). */
int kl_softmax(float* x, int n, void* stream);

/* ScaleSumKernel (KI:45-47; cpu/scale_sum_kernel.cpp:5-22): for d < size,
 * out[d] += scale[i] * value[i * stride + d] for i = 0 .. pos, in increasing i,
 * each product and each sum rounded to fp32 (bit-exact with the CPU path).
 * The rows of value may not overlap (stride >= size when pos > 0). */
int kl_scale_sum(const float* value, const float* scale, float* out, int pos, int size, int stride,
                 void* stream);

/* EmbeddingKernel (KI:16-17; cpu/emb_kernel.cpp:4-29, cuda/emb_kernel.cu:23-48):
 * out[i, :] = table[tokens[i], :] for i < n_tokens (no 512-token cap).
 * tokens is a DEVICE int32 array; ids outside [0, vocab) leave their row
 * untouched and set *bad_token_flag (device int32, may be NULL) to 1. */
int kl_embedding(const int32_t* tokens, int n_tokens, const float* table, int vocab, int dim,
                 float* out, int32_t* bad_token_flag, void* stream);

/* Measurement helper, no reference counterpart: the achievable HBM bandwidth
 * of this device, for comparing a kernel's rate with the box rather than
 * only with the 8 TB/s specification.  Allocates 2 * bytes (>= 1 MiB) of
 * device memory, then times `reps` passes (after one warm-up pass) of a
 * streaming read of all of it, one workgroup per CU on a contiguous chunk
 * each (*read_gbps: bytes read / s), and of a
 * device-to-device copy of one half into the other (*copy_gbps: bytes read +
 * written / s); frees everything before returning. */
int kl_hbm_probe(size_t bytes, int reps, float* read_gbps, float* copy_gbps);

/* Sampler::sample (include/sampler/sampler.h:10; argmax_sampler.cpp:5-13,
 * cuda/argmax_kernel.cu:73-87): first index of the maximum of x[0..n).  The
 * index is written to *out_index (device int32); workspace of
 * kl_argmax_workspace_size() bytes, zeroed once before first use. */
int kl_argmax_workspace_size(int n, size_t* bytes);
int kl_argmax(const float* x, int n, int32_t* out_index, void* workspace, size_t workspace_bytes,
              void* stream);

/* ---------------------------------------------------------------------------
 * Synthetic model images in the reference's .bin formats (the byte layouts
 * written by tools/export_llama.py:79-131 (fp32 v0), :134-210 (int8 g64),
 * tools/export_qwen2.py:79-134 (bias after each of wq/wk/wv), :137-210 (int8,
 * the Llama int8 layout) and tools/export_qwen3.py:55-102 (8-int header)).
 * Matrices, embeddings and biases are N(0, stddev) from a counter-based
 * generator keyed by (seed, tensor role, layer, element); norm weights are 1.0,
 * or 1 + N(0, norm_stddev) per norm role and layer; the unused freq tables of
 * the v0/Qwen2 layouts are written as zeros.  Host-only, no GPU needed.
 * ------------------------------------------------------------------------- */
typedef struct kl_model_spec {
  int32_t family;     /* KL_FAMILY_* */
  int32_t dim;        /* model width */
  int32_t q_dim;      /* heads * head_size (== dim except Qwen3) */
  int32_t hidden_dim; /* FFN width */
  int32_t layers;
  int32_t heads;
  int32_t kv_heads;
  int32_t vocab;
  int32_t seq_len;
  int32_t tied;       /* classifier = embedding (not for int8 or Qwen3) */
  int32_t group_size; /* 0: fp32 image; >0: int8 per-group image (Llama / Qwen2) */
  float norm_stddev;  /* 0: every norm weight 1.0; >0: 1 + N(0, norm_stddev) */
} kl_model_spec;

int kl_synth_image_size(const kl_model_spec* spec, int64_t* bytes);
int kl_synth_image(const kl_model_spec* spec, uint64_t seed, float stddev, void* out,
                   int64_t out_bytes, int n_threads);
/* The same N(0, stddev) stream for one tensor role/layer, for tests. */
int kl_synth_normal(uint64_t seed, int32_t role, int32_t layer, float stddev, float* out,
                    int64_t n);
/* The int8 quantiser of the image writer (export_llama.py:49-73). */
int kl_quantize_q8(const float* w, int64_t n, int group_size, int8_t* q, float* scales);

/* ---------------------------------------------------------------------------
 * Decode engine: the whole per-token step of model::LLama2Model /
 * Qwen2Model / Qwen3Model (source/model/llama3.cpp:146-166, :599-744;
 * qwen2.cpp:205-225, :640-801; qwen3.cpp:147-167, :459-640) on fused gfx950
 * kernels, replayed as one HIP graph per step.
 * ------------------------------------------------------------------------- */
typedef struct kl_engine kl_engine;

/* Parses a reference-format image (model/model.cpp:41-141 plus the loaders
 * model/llama3.cpp:183-422, qwen2.cpp:348-485, qwen3.cpp:186-299) from host
 * memory and uploads it to the current device.  quant != 0 selects the int8
 * layout.  The image may be freed after the call. */
int kl_engine_create(const void* image, size_t bytes, int family, int quant, kl_engine** out);
int kl_engine_destroy(kl_engine* e);
/* dims: {dim, q_dim, kv_dim, hidden, layers, heads, kv_heads, vocab, seq_len, head_size} */
int kl_engine_dims(const kl_engine* e, int32_t* out10);
int kl_engine_weight_bytes(const kl_engine* e, int64_t* bytes);
int kl_engine_set_graph(kl_engine* e, int enable);
/* Execution mode of the step.  KL_MODE_PERSISTENT (the default where the
 * device can hold one 512-thread workgroup per CU): one cooperative launch per
 * token runs every layer; workgroups hand activations to each other through
 * tagged stores (no grid barriers) and issue each phase's first weight loads
 * before they wait for its input.  The grid (one workgroup per CU) is launched
 * with hipLaunchKernel where the occupancy query shows it co-resident, else
 * cooperatively; every device-side wait is bounded and a timeout surfaces as
 * KL_EDEVICE (environment KL_PERSISTENT_LAUNCH=cooperative forces the
 * cooperative launch).  KL_MODE_MULTI: 5 kernels per layer plus the
 * classifier, replayed as a HIP graph (kl_engine_set_graph).
 * Both modes compute the same step; setting KL_MODE_PERSISTENT where it does
 * not fit returns KL_EUNSUPP. */
#define KL_MODE_PERSISTENT 0
#define KL_MODE_MULTI 1
int kl_engine_set_mode(kl_engine* e, int mode);
int kl_engine_get_mode(const kl_engine* e, int* mode);
/* Persistent-mode launch shape: workgroups, threads per workgroup, dynamic
 * LDS bytes. */
int kl_engine_launch_shape(const kl_engine* e, int32_t* workgroups, int32_t* threads,
                           int64_t* lds_bytes);
/* Model::predict (model/model.h:21-22, llama3.cpp:641-649): embed `token`,
 * run every layer at `pos`, final norm, classifier and argmax.  Blocks until
 * done; *next (may be NULL) receives the argmax, logits (host, may be NULL)
 * the vocab logits. */
int kl_engine_step(kl_engine* e, int32_t token, int32_t pos, int32_t* next, float* logits);
/* The demo/main.cpp:5-47 greedy loop entirely on the device: P prompt tokens
 * at positions 0..P-1, then n_new sampled tokens (out_tokens[n_new]).
 * *decode_ms (may be NULL) receives the device time of the n_new sampled
 * steps (positions P-1 .. P+n_new-2), measured with HIP events. */
int kl_engine_generate(kl_engine* e, const int32_t* prompt, int P, int n_new, int32_t* out_tokens,
                       float* decode_ms);
/* Benchmark run: like kl_engine_generate with n_warmup + n_timed sampled
 * tokens, where *timed_ms is the device time (HIP events on the engine's
 * stream) of the last n_timed steps only.  out_tokens[n_warmup + n_timed].
 * With kl_engine_set_prefill on (and n_warmup >= 1, P >= 2) the prompt runs
 * as one batched prefill, which also samples the first warm-up token; the
 * timed steps are at the same positions either way. */
int kl_engine_bench(kl_engine* e, const int32_t* prompt, int P, int n_warmup, int n_timed,
                    int32_t* out_tokens, float* timed_ms);
/* Batched prompt prefill: positions 0 .. P-1 of `prompt` through every layer
 * at once (row RMSNorm, MFMA GEMMs, batched q/k norm and RoPE, causal
 * attention, SwiGLU), K and V rows written to the caches, then the final norm,
 * classifier and argmax of position P-1: *next (may be NULL) receives the
 * greedy token, logits (host, may be NULL) the vocab logits of position P-1.
 * Same result as P kl_engine_step calls up to float rounding; a following
 * kl_engine_step(e, *next, P, ...) continues the sequence.  Chunks of at most
 * 1024 positions.  KL_EUNSUPP for head sizes other than 32, 64, 128 (and for
 * int8 images whose dimensions are not whole 32-column blocks).  Blocks until
 * done; *prefill_ms (may be NULL) receives its device time. */
int kl_engine_prefill(kl_engine* e, const int32_t* prompt, int P, int32_t* next, float* logits,
                      float* prefill_ms);
/* When enabled (default off), kl_engine_generate runs prompts of 2 or more
 * tokens through kl_engine_prefill; out_tokens[0] is then the prefill's token
 * and *decode_ms covers the n_new - 1 decode steps that follow.  Returns
 * KL_EUNSUPP (and stays off) where the prefill does not support the model. */
int kl_engine_set_prefill(kl_engine* e, int enable);

/* Per-kernel timing: runs `steps` decode steps from (token, pos0) without the
 * graph, with a HIP event recorded between consecutive launches on the
 * engine's stream, and returns the average duration and launch count per
 * kernel kind: [embed, qkv, attn, wo, w13, w2, cls, step]; in the persistent
 * mode only `step` (the whole-token kernel) is used. */
int kl_engine_profile(kl_engine* e, int32_t token, int32_t pos0, int steps, float* avg_ms8,
                      int32_t* counts8);
/* Device-time trace of one persistent step (the reference's per-op profile,
 * model/qwen2.cpp:16-68, measured on the device): runs the step for (token,
 * pos) and returns ticks of the 100 MHz s_memrealtime clock, slot-major
 * [n_slots][n_workgroups]: slot 0 = kernel entry; phase p (5 per layer: QKV,
 * attention, WO, W1/W3, W2; then the classifier) has slot 2p+1 = its input
 * staged and slot 2p+2 = its outputs stored.  Unused slots are 0.  KL_EUNSUPP outside the persistent mode; KL_EWORKSPACE when
 * max_ticks < n_slots * n_workgroups (the sizes are still returned). */
int kl_engine_trace_step(kl_engine* e, int32_t token, int32_t pos, uint64_t* ticks,
                         int64_t max_ticks, int32_t* n_slots, int32_t* n_workgroups);
/* Device pointers for inspection: logits [vocab], key/value caches
 * [layers][seq_len][kv_dim]. */
int kl_engine_buffers(const kl_engine* e, const float** logits, const float** key_cache,
                      const float** value_cache);
/* Stream the engine launches on (a hipStream_t as void*). */
int kl_engine_stream(const kl_engine* e, void** stream);

#ifdef __cplusplus
}
#endif
#endif /* KUIPER_HIP_H_ */
