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
// r % 4][l % 32]).  K advances in blocks of 32 staged in LDS (double
// buffered, one barrier per block, the next block's global loads in flight
// during the current block's 16 MFMAs).  Inside a block the 32 k indices are
// visited in the order that lets each lane fetch its 16 operands of a block
// with four ds_read_b128: MFMA step s uses, in lane l, column 16 (l / 32) + s.
// The same permutation applies to both operands, so every product
// A[m][k] W[n][k] is formed exactly once.  (Measured at the Qwen3-4B prefill
// shapes, M = 512: blocks of 32 are 3-7% faster than 16; 64 x 64 tiles of four
// waves beat 128 x 64, 64 x 128 and 128 x 128 tiles, which leave too few
// workgroups; two accumulators per wave or loads two blocks ahead change
// nothing.)
//
// Grouped launches compute up to three outputs over the same A (the Q, K and V
// projections) in one grid, and split-K divides the K blocks among
// blockIdx.y with a fixed-order reduction, so that narrow outputs (few tiles)
// still fill the chip.
//
// int8 weights (Q8): W holds int8 [N x ldw] with one fp32 scale per 2^gshift
// consecutive elements of the flattened matrix (the image's group-wise
// layout, export_llama.py:49-73).  Each thread loads the 4 bytes that stand in
// for one float4 of the fp32 path and its group's scale, and stores
// float(q) * scale to LDS (the dequantised weight of the reference's int8
// GEMV, cuda/matmul_kernel.cu:73); the MFMA loop is the same.  K must be a
// whole number of blocks.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gemm_run.hpp"

namespace kl {

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef float gf16 __attribute__((ext_vector_type(16)));

template <int WM, int WN, int TM, int TN, bool Q8 = false>
__global__ __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(3))) void k_gemm_f32(
    GemmArgs g) {
  constexpr int BM = WM * TM * 32, BN = WN * TN * 32, BK = kGemmBK, LDK = kGemmLDK;
  constexpr int NT = WM * WN * 64;
  constexpr int A4 = BM * BK / 4, W4 = BN * BK / 4;  // float4s per tile
  constexpr int LA = (A4 + NT - 1) / NT, LW = (W4 + NT - 1) / NT;
  __shared__ __align__(16) float As[2][BM * LDK];
  __shared__ __align__(16) float Ws[2][BN * LDK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  // Segment of this tile (uniform per workgroup).
  int sidx = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < g.nseg && static_cast<int>(blockIdx.x) >= g.seg[i].tile0) sidx = i;
  const float* __restrict__ A = g.A;
  const void* W = g.seg[0].W;
  float* C = g.seg[0].C;
  const float* bias = g.seg[0].bias;
  const float* S = g.seg[0].S;
  int N = g.seg[0].N, ldw = g.seg[0].ldw, ldc = g.seg[0].ldc, tile0 = 0, gshift = g.seg[0].gshift;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i == sidx) {
      W = g.seg[i].W;
      C = g.seg[i].C;
      bias = g.seg[i].bias;
      S = g.seg[i].S;
      N = g.seg[i].N;
      ldw = g.seg[i].ldw;
      ldc = g.seg[i].ldc;
      tile0 = g.seg[i].tile0;
      gshift = g.seg[i].gshift;
    }
  const int M = g.M, K = g.K, lda = g.lda;
  // Tiles along M are adjacent in launch order, so the workgroups that share
  // a W tile run together and read it from cache.
  const int local = static_cast<int>(blockIdx.x) - tile0;
  const int tm = local % g.tiles_m, tn = local / g.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  // K range of this split, in whole blocks.
  const int nkt = (K + BK - 1) / BK;
  const int kb0 = static_cast<int>(blockIdx.y) * nkt / g.splits;
  const int kb1 = (static_cast<int>(blockIdx.y) + 1) * nkt / g.splits;

  // The next block's loads land in ra/rw while the current block's MFMAs run.
  // The steady state spends almost no vector instructions on addressing: each
  // load is a per-thread 32-bit byte offset (fixed for the whole K loop) from a
  // uniform base that advances by one block, and each LDS store address is
  // fixed.  Rows past M or N are clamped to the last row instead of masked:
  // they only feed outputs that are never stored.  Only a partial last block
  // (K not a multiple of BK) zeroes columns past K, in both operands.
  static_assert(A4 % NT == 0 && W4 % NT == 0, "whole float4 loads per thread");
  gf4 ra[LA], rw[LW];
  int rq[LW];     // int8: four weights per thread and load
  float rs[LW];   // int8: their group's scale
  unsigned int offa[LA], offw[LW], colok_a[LA], colok_w[LW];
  unsigned int lofa[LA], lofw[LW];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int idx = tid + i * NT;
    const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
    const int m = min(m0 + r, M - 1);
    offa[i] = static_cast<unsigned int>((m * lda + c) * 4);
    colok_a[i] = static_cast<unsigned int>(c);
    lofa[i] = static_cast<unsigned int>(r * LDK + c);
  }
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    const int idx = tid + i * NT;
    const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
    const int n = min(n0 + r, N - 1);
    // fp32: byte offset; int8: element (= byte) offset.
    offw[i] = static_cast<unsigned int>((n * ldw + c) * (Q8 ? 1 : 4));
    colok_w[i] = static_cast<unsigned int>(c);
    lofw[i] = static_cast<unsigned int>(r * LDK + c);
  }
  auto gload = [&](int k0) {
    const char* ba = reinterpret_cast<const char*>(A) + static_cast<size_t>(k0) * 4;
    const char* bw = reinterpret_cast<const char*>(W) + static_cast<size_t>(k0) * (Q8 ? 1 : 4);
    if constexpr (Q8) {  // whole blocks only
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const gf4*>(ba + offa[i]);
#pragma unroll
      for (int i = 0; i < LW; ++i) {
        rq[i] = *reinterpret_cast<const int*>(bw + offw[i]);
        rs[i] = S[(offw[i] + static_cast<unsigned int>(k0)) >> gshift];
      }
    } else if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const gf4*>(ba + offa[i]);
#pragma unroll
      for (int i = 0; i < LW; ++i) rw[i] = *reinterpret_cast<const gf4*>(bw + offw[i]);
    } else {  // partial last block: columns past K read column k0 and are zeroed
      const gf4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < LA; ++i) {
        const bool ok = k0 + static_cast<int>(colok_a[i]) < K;
        ra[i] = *reinterpret_cast<const gf4*>(ba + offa[i] - (ok ? 0u : colok_a[i] * 4));
        if (!ok) ra[i] = z;
      }
#pragma unroll
      for (int i = 0; i < LW; ++i) {
        const bool ok = k0 + static_cast<int>(colok_w[i]) < K;
        rw[i] = *reinterpret_cast<const gf4*>(bw + offw[i] - (ok ? 0u : colok_w[i] * 4));
        if (!ok) rw[i] = z;
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LA; ++i) *reinterpret_cast<gf4*>(&As[buf][lofa[i]]) = ra[i];
    if constexpr (Q8) {
#pragma unroll
      for (int i = 0; i < LW; ++i) {
        const int q = rq[i];
        const gf4 w = {static_cast<float>((q << 24) >> 24) * rs[i], static_cast<float>((q << 16) >> 24) * rs[i],
                       static_cast<float>((q << 8) >> 24) * rs[i], static_cast<float>(q >> 24) * rs[i]};
        *reinterpret_cast<gf4*>(&Ws[buf][lofw[i]]) = w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < LW; ++i) *reinterpret_cast<gf4*>(&Ws[buf][lofw[i]]) = rw[i];
    }
  };

  gf16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = gf16{};

  if (kb0 < kb1) {
    gload(kb0 * BK);
    sstore(0);
  }
  __syncthreads();
  constexpr int KH = BK / 2;       // columns of a k block per lane half
  constexpr int NR = KH / 4;       // float4 reads per operand
  const int kc = KH * (lane >> 5);  // this lane's KH columns of a k block
  for (int kt = kb0; kt < kb1; ++kt) {
    const int cur = (kt - kb0) & 1;
    if (kt + 1 < kb1) gload((kt + 1) * BK);
    gf4 af[TM][NR], bf[TN][NR];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const float* p = &As[cur][(wm * TM * 32 + a * 32 + (lane & 31)) * LDK + kc];
#pragma unroll
      for (int j = 0; j < NR; ++j) af[a][j] = *reinterpret_cast<const gf4*>(p + 4 * j);
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float* p = &Ws[cur][(wn * TN * 32 + b * 32 + (lane & 31)) * LDK + kc];
#pragma unroll
      for (int j = 0; j < NR; ++j) bf[b][j] = *reinterpret_cast<const gf4*>(p + 4 * j);
    }
#pragma unroll
    for (int s = 0; s < KH; ++s)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][s >> 2][s & 3],
                                                           bf[b][s >> 2][s & 3], acc[a][b], 0, 0, 0);
    if (kt + 1 < kb1) sstore(cur ^ 1);
    __syncthreads();
  }

  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * M * N : nullptr;
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
          if (wsp) {
            wsp[static_cast<size_t>(m) * N + n] = v;
          } else {
            if (bias) v += bias[n];
            float* cp = C + static_cast<size_t>(m) * ldc + n;
            if (g.accumulate) v = *cp + v;
            *cp = v;
          }
        }
      }
}

// C = sum of the split partials in split order (+ bias) (+ C).
__global__ void k_gemm_reduce(const float* __restrict__ ws, int splits, int M, int N,
                              float* __restrict__ C, int ldc, const float* __restrict__ bias,
                              int accumulate) {
  const size_t total = static_cast<size_t>(M) * N;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    float v = ws[i];
    for (int s = 1; s < splits; ++s) v += ws[static_cast<size_t>(s) * total + i];
    const int m = static_cast<int>(i / N), n = static_cast<int>(i - static_cast<size_t>(m) * N);
    if (bias) v += bias[n];
    float* cp = C + static_cast<size_t>(m) * ldc + n;
    if (accumulate) v = *cp + v;
    *cp = v;
  }
}

}  // namespace kl
