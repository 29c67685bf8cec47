// fp32 GEMM on the gfx950 matrix cores for the batched prompt prefill:
//   C[M x N] (+)= A[M x K] . W[N x K]^T (+ bias[N])
// A holds one token per row (activations), W is a weight matrix exactly as the
// model image stores it ([out x in], row-major), so both operands are
// K-contiguous.  The reference has no batched path (MatmulLayer takes a 1-D
// input, op/matmul.cpp:20; the prompt runs token by token, demo/main.cpp:20-22).
//
// Tiling: a workgroup of WM x WN waves computes a (WM*TM*32) x (WN*TN*32) tile
// of C; each wave owns TM x TN blocks of 32 x 32 accumulated with
// v_mfma_f32_32x32x2f32 (A operand: lane l holds A[l % 32][k], B operand:
// W[l % 32][k], result register r of lane l is C[8 (r / 4) + 4 (l / 32) +
// r % 4][l % 32]).  K advances in blocks of 16 staged in LDS (double
// buffered, one barrier per block, the next block's global loads in flight
// during the current block's MFMAs).  Inside a block the 16 k indices are
// visited in the order that lets each lane fetch its 8 operands of a block
// with two ds_read_b128: MFMA step s uses, in lane l, column 8 (l / 32) + s.
// The same permutation applies to both operands, so every product
// A[m][k] W[n][k] is formed exactly once.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace kl {

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef float gf16 __attribute__((ext_vector_type(16)));

constexpr int kGemmBK = 16;
constexpr int kGemmLDK = kGemmBK + 4;  // padded LDS row (floats)

template <int WM, int WN, int TM, int TN>
__global__ __launch_bounds__(WM * WN * 64) void k_gemm_f32(
    const float* __restrict__ A, const float* __restrict__ W, float* __restrict__ C,
    const float* __restrict__ bias, int M, int N, int K, int lda, int ldw, int ldc,
    int accumulate, int tiles_m) {
  constexpr int BM = WM * TM * 32, BN = WN * TN * 32, BK = kGemmBK, LDK = kGemmLDK;
  constexpr int NT = WM * WN * 64;
  constexpr int A4 = BM * BK / 4, W4 = BN * BK / 4;  // float4s per tile
  constexpr int LA = (A4 + NT - 1) / NT, LW = (W4 + NT - 1) / NT;
  __shared__ __align__(16) float As[2][BM * LDK];
  __shared__ __align__(16) float Ws[2][BN * LDK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  // Tiles along M are adjacent in launch order, so the workgroups that share
  // a W tile run together and read it from cache.
  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  gf4 ra[LA], rw[LW];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + i * NT;
      const int r = idx >> 2, c = (idx & 3) * 4;
      const int m = m0 + r, k = k0 + c;
      const bool ok = idx < A4 && m < M && k < K;
      const gf4 v = *reinterpret_cast<const gf4*>(A + static_cast<size_t>(ok ? m : 0) * lda +
                                                  (ok ? k : 0));
      ra[i] = ok ? v : gf4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const int idx = tid + i * NT;
      const int r = idx >> 2, c = (idx & 3) * 4;
      const int n = n0 + r, k = k0 + c;
      const bool ok = idx < W4 && n < N && k < K;
      const gf4 v = *reinterpret_cast<const gf4*>(W + static_cast<size_t>(ok ? n : 0) * ldw +
                                                  (ok ? k : 0));
      rw[i] = ok ? v : gf4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + i * NT;
      if (idx < A4) *reinterpret_cast<gf4*>(&As[buf][(idx >> 2) * LDK + (idx & 3) * 4]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      const int idx = tid + i * NT;
      if (idx < W4) *reinterpret_cast<gf4*>(&Ws[buf][(idx >> 2) * LDK + (idx & 3) * 4]) = rw[i];
    }
  };

  gf16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = gf16{};

  const int nk = (K + BK - 1) / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int kc = 8 * (lane >> 5);  // this lane's 8 columns of a k block
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    gf4 af[TM][2], bf[TN][2];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const float* p = &As[cur][(wm * TM * 32 + a * 32 + (lane & 31)) * LDK + kc];
      af[a][0] = *reinterpret_cast<const gf4*>(p);
      af[a][1] = *reinterpret_cast<const gf4*>(p + 4);
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float* p = &Ws[cur][(wn * TN * 32 + b * 32 + (lane & 31)) * LDK + kc];
      bf[b][0] = *reinterpret_cast<const gf4*>(p);
      bf[b][1] = *reinterpret_cast<const gf4*>(p + 4);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][s >> 2][s & 3],
                                                           bf[b][s >> 2][s & 3], acc[a][b], 0, 0, 0);
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * TM * 32 + a * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int n = n0 + wn * TN * 32 + b * 32 + (lane & 31);
        if (m < M && n < N) {
          float v = acc[a][b][r];
          if (bias) v += bias[n];
          float* cp = C + static_cast<size_t>(m) * ldc + n;
          if (accumulate) v = *cp + v;
          *cp = v;
        }
      }
}

}  // namespace kl
