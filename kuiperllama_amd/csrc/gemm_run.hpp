// The prefill GEMM's launch interface (kernel in gemm.hpp, launcher in
// ops.hip): what a caller outside ops.hip needs to run it with fp32 or int8
// weight segments.
#pragma once
#include <hip/hip_runtime.h>

namespace kl {

constexpr int kGemmBK = 32;
constexpr int kGemmLDK = kGemmBK + 4;  // padded LDS row (floats)
constexpr int kGemmMaxSeg = 3;

// One output of a grouped GEMM: C_s = A . W_s^T (+ bias_s) over the same A.
struct GemmSeg {
  const void* W;     // fp32, or int8 with scales S
  float* C;
  const float* bias;
  int N, ldw, ldc;
  int tile0;         // first workgroup tile of this segment
  const float* S;    // int8 group scales (nullptr: fp32 weights)
  int gshift;        // int8 group size = 1 << gshift
  size_t wsoff;      // split-K: this output's [M][N] partials within a split's slab
};

struct GemmArgs {
  const float* A;
  int M, K, lda;
  int accumulate;  // C += product (else C = product)
  int tiles_m;
  int nseg;
  GemmSeg seg[kGemmMaxSeg];
  // Split-K: blockIdx.y = split; the partial products of output s go to
  // ws + split * ws_split + seg[s].wsoff ([M][N_s]) and k_gemm_reduce applies
  // bias and accumulate.
  float* ws;
  size_t ws_split;  // floats per split: M * (N_0 + N_1 + ...)
  int splits;
};

// Operands of the split-product GEMM (k_gemm_x6): A (M x K) and every W_s
// (N_s x K) as three bf16 planes in the tiled plane format of k_split3
// (x6_tile_offset, gemm.hpp).
struct GemmX6Planes {
  const void* A;
  const void* W[kGemmMaxSeg];
  int w_planes;  // 1: every W's planes 1 and 2 are zero (bf16-exact weights); 0 or 3: all three
};

struct GemmX6Args {
  GemmArgs g;
  GemmX6Planes p;
  int tiles;  // 128 x 128 tiles over every output (the grid is padded to a multiple of 8)
};

// Short int8 prompts (k_gemm_q8s): one output over prepacked weights P
// (k_q8s_pack); wg0 = first workgroup of the output.
struct GemmQ8sSeg {
  const void* P;
  float* C;
  const float* bias;
  int N, ldc, wg0;
  size_t wsoff;
};

struct GemmQ8sArgs {
  const void* A;  // activation planes (k_q8s_split)
  int M, K, gshift, accumulate, nseg, splits;
  GemmQ8sSeg seg[kGemmMaxSeg];
  float* ws;
  size_t ws_split;
};

// Host launcher (ops.hip): C_s (+)= A . W_s^T (+ bias_s) for nseg outputs in
// one grid; splits > 1 divides K among blockIdx.y into ws (splits * M *
// (N_0 + ...) floats) and reduces in split order.  Every segment is fp32 or
// every one int8.
int gemm_run(const float* A, int M, int K, int lda, int nseg, const GemmSeg* segs, int accumulate,
             float* ws, int splits, hipStream_t st);

// Host launcher (ops.hip) of k_gemm_x6: the same products from bf16 planes
// (segs[s].W and ldw unused).  K a multiple of 32.  Chooses the split count
// itself (up to 8, where ws_bytes holds splits * M * (N_0 + ...) floats).
// With `deferred`, a split-K launch leaves its partials in ws (no reduction:
// the caller's next producer sums them) and *deferred = the split count (1:
// C was written directly).
int gemm_run_x6(const GemmX6Planes& planes, int M, int K, int nseg, const GemmSeg* segs,
                int accumulate, float* ws, size_t ws_bytes, hipStream_t st, int* deferred = nullptr);

// Host launcher (ops.hip) of k_split3: rows x cols fp32 (stride ldx, cols a
// multiple of 32) into the tiled planes (x6_plane_bytes(rows, cols) bytes).
// *flag |= 1 if planes 1 or 2 of a rows x K matrix in the tiled plane format
// hold a nonzero bit (so the matrix needs all three planes; else plane 0 is
// the matrix exactly).  Asynchronous; *flag must start at 0.
int x6_planes_flag_run(const void* planes, int rows, int K, unsigned* flag, hipStream_t st);
int split3_run(const float* x, int rows, int cols, int ldx, void* planes, hipStream_t st);

// Short int8 prompts: bytes of a prepacked int8 matrix (q8s_pack_run) and of
// the activation planes (q8s_split_run, 32 rows); the launcher over nseg
// outputs of the same A (segs[s].W: the packed matrix), splits chosen within
// ws_bytes; M <= 32, group size 32 or 64 dividing K.
size_t q8s_packed_bytes(int N, int K, int group_size);
inline size_t q8s_aplane_bytes(int K) { return static_cast<size_t>(K) * 32 * 3 * 2; }
int q8s_pack_run(const int8_t* q, const float* scales, int N, int K, int group_size, void* packed,
                 hipStream_t st);
int q8s_split_run(const float* A, int M, int K, int lda, void* planes, hipStream_t st);
int gemm_run_q8s(const void* planes, int M, int K, int group_size, int nseg, const GemmSeg* segs,
                 int accumulate, float* ws, size_t ws_bytes, hipStream_t st, int* deferred = nullptr);

// GEMM-input producers (ops.hip) writing the operand planes directly (q8s:
// k_gemm_q8s's lane order, rows <= 32; else the tiled format):
// norm_planes_run: x += sum of `splits` partial slabs (ws + z ws_split, rows
// x n; none for splits = 0), written back, then RMSNorm(x) * w into planes;
// swiglu_planes_run: silu(h1) * h3 into planes, h1 and h3 the sums of the
// partial slabs at ws (+ wsoff3 for h3) when splits > 0.
int norm_planes_run(float* x, const float* w, int rows, int n, float eps, const float* ws, int splits,
                    size_t ws_split, void* planes, bool q8s, hipStream_t st);
int swiglu_planes_run(const float* h1, const float* h3, int rows, int F, const float* ws, int splits,
                      size_t ws_split, size_t wsoff3, void* planes, bool q8s, hipStream_t st);
// The partials of a grouped Q/K/V launch over n rows left unsummed (segments q
// [n x dim], k and v [n x kv_dim] at ws + z ws_split): q, k and v summed in
// split order plus their biases (k_gemm_reduce's arithmetic), q and k rotated
// at positions pos0 + r (kl_rope_rows's rotation), all three stored.
int qkv_sum_rope_run(int style, int dim, int kv_dim, int hd, const float* ws, int splits, size_t ws_split,
                     const float* bq, const float* bk, const float* bv, float* q, int ldq, float* k, int ldk,
                     float* v, int ldv, int pos0, int n, const float* sin_t, const float* cos_t,
                     hipStream_t st);
// x[rows x n] += the sum of `splits` partial slabs of rows x n at ws (k_gemm_reduce).
int partials_add_run(float* x, int rows, int n, const float* ws, int splits, hipStream_t st);

inline size_t x6_plane_bytes(int rows, int cols) {
  return static_cast<size_t>((rows + 15) / 16) * 16 * cols * 3 * 2;
}

}  // namespace kl
