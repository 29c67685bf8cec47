// fp32 GEMM on the gfx950 matrix cores for the batched prompt prefill:
//   C[M x N] (+)= A[M x K] . W[N x K]^T (+ bias[N])
// A holds one token per row (activations), W is a weight matrix exactly as the
// model image stores it ([out x in], row-major), so both operands are
// K-contiguous.  The reference has no batched path (MatmulLayer takes a 1-D
// input, op/matmul.cpp:20; the prompt runs token by token, demo/main.cpp:20-22).
//
// Four kernels share the launch arguments (GemmArgs, gemm_run.hpp; k_gemm_x6
// wraps them with its operand planes): k_gemm_f32_dma (fp32), k_gemm_f32
// (int8 and other K) and k_gemm_q8_dma (int8, at most 32 rows), four waves per
// workgroup, and k_gemm_x6 (fp32 operands as bf16 planes on the bf16 matrix
// cores; four or eight waves).  k_gemm_q8s (int8 weights prepacked in lane
// order, at most 32 rows, eight waves) has arguments of its own.  The last
// three are described at their definitions.
//
// k_gemm_f32_dma<TA> (fp32 weights, K a multiple of 32; every model
// projection): a workgroup tile of 32 TA x 64 (TA = 2: 64 x 64, three
// workgroups per CU; TA = 4: 128 x 64, two per CU, for launches with at least
// 1024 such tiles, where halving the operand reads and barriers per MFMA pays
// for the fewer resident waves: +6% on the Qwen3-4B W1/W3 shape at 512 rows, -5 to -13% on
// the narrower ones); each wave owns TA x 2 blocks of 16 x 16 accumulated with
// v_mfma_f32_16x16x4f32 (A operand: lane l holds A[l % 16][k], B operand
// W[l % 16][k], k = l / 16; result register r of lane l is
// C[4 (l / 16) + r][l % 16]).  K advances in blocks of 32 columns staged in
// LDS by direct-to-LDS loads (global_load_lds_dwordx4: no VGPR staging, no LDS
// store instructions) through a 3-stage ring, block k + 2 requested while
// block k is computed, one barrier per block.  A 1 KB load instruction of a
// wave fills 8 rows of 128 B; chunk q (16 B) of row r sits in slot
// q ^ dma_swz(r), which each lane gets by loading the chunk that belongs in
// its slot, so the operand reads are conflict-free without padding.  Lane group
// g = l / 16 takes k columns 8 g .. 8 g + 7 of a block (two contiguous 16 B
// reads per row; A and W use the same permutation, so every product
// A[m][k] W[n][k] is formed exactly once).  The next block's operands are read
// into the other register buffer right after the barrier, while the current
// block's last two k steps run; the loop is unrolled by two so the buffers
// alternate without copies.  Measured on the Qwen3-4B prefill shapes (M = 512,
// one box): 107-121 TFLOP/s against 87-107 for k_gemm_f32 below; 2 x 2 waves of
// 32 x 32 with 16 x 16 blocks beat 32 x 32 blocks (v_mfma_f32_32x32x2f32),
// larger tiles (fewer workgroups at M = 512), a K depth of 64 (one workgroup
// per CU) and a hand-pinned schedule.
//
// k_gemm_f32 (int8 weights, and K not a multiple of 32): each wave owns one
// 32 x 32 block of v_mfma_f32_32x32x2f32 (A operand: lane l holds A[l % 32][k],
// B operand W[l % 32][k], result register r of lane l is C[8 (r / 4) +
// 4 (l / 32) + r % 4][l % 32]); K in blocks of 32 through double-buffered,
// padded LDS stored from registers (the next block's global loads in flight
// during the current block's 16 MFMAs); MFMA step s uses, in lane l, column
// 16 (l / 32) + s, so each lane fetches its 16 operands of a block with four
// ds_read_b128.
//
// Grouped launches compute up to three outputs over the same A (the Q, K and V
// projections) in one grid, and split-K divides the K blocks among
// blockIdx.y with a fixed-order reduction, so that narrow outputs (few tiles)
// still fill the chip.  Tiles along M are adjacent in launch order.
//
// int8 weights (Q8, k_gemm_f32): W holds int8 [N x ldw] with one fp32 scale per
// 2^gshift consecutive elements of the flattened matrix (the image's group-wise
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
  size_t wsoff = 0;
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
      wsoff = g.seg[i].wsoff;
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

  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * g.ws_split + wsoff : nullptr;
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

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

constexpr int kDmaStages = 3;

// Chunk swizzle of the direct-to-LDS tiles (rows of 128 B = 8 chunks of
// 16 B; chunk q of row r sits in slot q ^ dma_swz(r)).  A 16-byte LDS read
// is served half a wave at a time over 512 B of banks, i.e. the 32 lanes of
// a half wave (16 consecutive rows, two chunks c and c ^ 2 each) must land in
// 32 distinct 16-byte slots modulo 512 B: rows r, r + 4, r + 8, r + 12 share
// their position within 512 B, so bits 0 and 2 of the swizzle must follow
// r / 4 (bits 2 and 3 of r) and bit 1 may follow bit 1 of r.  r & 7 (the
// plain XOR) leaves rows r and r + 8 on the same slots: 2-way conflicts on
// every operand read (SQ_LDS_BANK_CONFLICT 1.05e9 -> 0 on the Qwen3-4B 512-row shapes).
__device__ __forceinline__ int dma_swz(int r) { return ((r >> 2) & 1) | (r & 2) | ((r >> 1) & 4); }

template <int TA>
__global__ __launch_bounds__(256) void k_gemm_f32_dma(GemmArgs g) {
  static_assert(TA == 2 || TA == 4, "wave tile rows: 32 or 64");
  constexpr int BM = 32 * TA, BN = 64, BK = 32;
  constexpr int SA = BM * BK, SW = BN * BK;   // floats per stage and operand
  constexpr int LI = BM / 8 / 4;              // 1 KB load instructions per wave: A
  constexpr int LW = BN / 8 / 4;              //   and W
  __shared__ __align__(1024) float L[kDmaStages * (SA + SW)];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  int sidx = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < g.nseg && static_cast<int>(blockIdx.x) >= g.seg[i].tile0) sidx = i;
  const float* __restrict__ A = g.A;
  const void* W = g.seg[0].W;
  float* C = g.seg[0].C;
  const float* bias = g.seg[0].bias;
  int N = g.seg[0].N, ldw = g.seg[0].ldw, ldc = g.seg[0].ldc, tile0 = 0;
  size_t wsoff = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i == sidx) {
      W = g.seg[i].W;
      C = g.seg[i].C;
      bias = g.seg[i].bias;
      N = g.seg[i].N;
      ldw = g.seg[i].ldw;
      ldc = g.seg[i].ldc;
      tile0 = g.seg[i].tile0;
      wsoff = g.seg[i].wsoff;
    }
  const int M = g.M, K = g.K, lda = g.lda;
  const int local = static_cast<int>(blockIdx.x) - tile0;
  const int tm = local % g.tiles_m, tn = local / g.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nkt = K / BK;
  const int kb0 = static_cast<int>(blockIdx.y) * nkt / g.splits;
  const int kb1 = (static_cast<int>(blockIdx.y) + 1) * nkt / g.splits;

  // Load instruction i of this wave fills tile rows 8 j .. 8 j + 7
  // (j = LI * wave + i); lane l writes slot l % 8 of row r = 8 j + l / 8,
  // which holds chunk (l % 8) ^ dma_swz(r).  Rows past M or N read the last
  // row (they only feed outputs that are never stored).
  unsigned int ga[LI], gw[LW];
#pragma unroll
  for (int i = 0; i < LI; ++i) {
    const int r = 8 * (LI * wave + i) + (lane >> 3);
    ga[i] = static_cast<unsigned int>((min(m0 + r, M - 1) * lda + 4 * ((lane & 7) ^ dma_swz(r))) * 4);
  }
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    const int r = 8 * (LW * wave + i) + (lane >> 3);
    gw[i] = static_cast<unsigned int>((min(n0 + r, N - 1) * ldw + 4 * ((lane & 7) ^ dma_swz(r))) * 4);
  }
  auto request = [&](int kb, int st) {
    const char* ba = reinterpret_cast<const char*>(A) + static_cast<size_t>(kb) * BK * 4;
    const char* bw = reinterpret_cast<const char*>(W) + static_cast<size_t>(kb) * BK * 4;
    float* la = L + st * (SA + SW);
    float* lw = la + SA;
#pragma unroll
    for (int i = 0; i < LI; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t*)(ba + ga[i]),
                                       (lds_void_t*)(la + 256 * (LI * wave + i)), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < LW; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t*)(bw + gw[i]),
                                       (lds_void_t*)(lw + 256 * (LW * wave + i)), 16, 0, 0);
  };
  // Operands: lane group g4 = l / 16 reads chunks 2 g4 and 2 g4 + 1 of rows
  // 16 TA wm + 16 a + l % 16 (A) and 32 wn + 16 b + l % 16 (W).
  const int g4 = lane >> 4, r16 = lane & 15;
  const int rowa = 16 * TA * wm + r16, rowb = 32 * wn + r16;
  int oa[2], ob[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    oa[j] = rowa * BK + 4 * ((2 * g4 + j) ^ dma_swz(rowa));
    ob[j] = rowb * BK + 4 * ((2 * g4 + j) ^ dma_swz(rowb));
  }
  gf4 af[2][TA][2], bf[2][2][2];  // [register buffer][block][16-byte read]
  auto operands = [&](int st, int p) {
    const float* la = L + st * (SA + SW);
    const float* lw = la + SA;
#pragma unroll
    for (int a = 0; a < TA; ++a)
#pragma unroll
      for (int j = 0; j < 2; ++j) af[p][a][j] = *reinterpret_cast<const gf4*>(la + a * 16 * BK + oa[j]);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[p][b][j] = *reinterpret_cast<const gf4*>(lw + b * 16 * BK + ob[j]);
  };
  gf4 acc[TA][2];
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = gf4{0.f, 0.f, 0.f, 0.f};
  auto steps = [&](int p, int s0, int s1) {
#pragma unroll
    for (int s = s0; s < s1; ++s)
#pragma unroll
      for (int a = 0; a < TA; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[p][a][s >> 2][s & 3], bf[p][b][s >> 2][s & 3],
                                                           acc[a][b], 0, 0, 0);
  };
  constexpr int kLoads = LI + LW;  // load instructions per block and wave
  if (kb0 < kb1) {
    // Blocks kb0 and kb0 + 1 in flight, block kb0 landed in every wave.
    request(kb0, 0);
    request(min(kb0 + 1, kb1 - 1), 1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads) : "memory");
    __builtin_amdgcn_s_barrier();
    operands(0, 0);
    int st = 0;
    // Block kt with its operands in register buffer p: request block kt + 2
    // into the stage block kt - 1 used, run 6 of the 8 k steps, wait until
    // block kt + 1 has landed (only the newest request may be outstanding)
    // and every wave is done reading, then read block kt + 1's operands into
    // buffer p ^ 1 while the last 2 steps run.  The last blocks request
    // themselves again (a stage nobody reads afterwards).
    auto block = [&](int kt, int p) {
      const int sn = st == 0 ? 2 : st - 1;
      const int st1 = st == 2 ? 0 : st + 1;
      request(min(kt + 2, kb1 - 1), sn);
      steps(p, 0, 6);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(kLoads) : "memory");
      __builtin_amdgcn_s_barrier();
      operands(st1, p ^ 1);
      steps(p, 6, 8);
      st = st1;
    };
    int kt = kb0;
    for (; kt + 1 < kb1; kt += 2) {
      block(kt, 0);
      block(kt + 1, 1);
    }
    if (kt < kb1) block(kt, 0);
  }

  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * g.ws_split + wsoff : nullptr;
#pragma unroll
  for (int a = 0; a < TA; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * TA * wm + 16 * a + 4 * g4 + r;
        const int n = n0 + 32 * wn + 16 * b + r16;
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

// k_gemm_q8_dma (int8 weights, at most 32 rows, group size >= 32): the
// direct-to-LDS pipeline of k_gemm_f32_dma for a 32 x 128 tile, with the
// weights staged as int8.  Per 32-column block a 3-stage ring holds the A tile
// (32 rows of 128 B, chunks swizzled by dma_swz), the W tile (128 rows of
// 32 B) and each W row's group scale (one per row and block: the block lies in
// one group); every wave issues one direct-to-LDS load of each per block (its
// 8 A rows, its 32 W rows, its 32 scales), so the wait counts are uniform.
// Wave w owns columns 32 w .. 32 w + 31 as 2 x 2 blocks of 16 x 16
// (v_mfma_f32_16x16x4f32); lane group g4 = l / 16 takes k = 8 g4 .. 8 g4 + 7
// of a block: two 16-byte A reads per row block and one 8-byte read of its
// weights per column block, dequantised in registers as float(q) * scale (the
// reference int8 GEMV's weight, cuda/matmul_kernel.cu:73).  A quarter of the
// LDS traffic of staging dequantised floats, and no register staging.
__global__ __launch_bounds__(256) void k_gemm_q8_dma(GemmArgs g) {
  constexpr int BM = 32, BN = 128, BK = 32;
  constexpr int SA = BM * BK;        // A floats per stage
  constexpr int SW = BN * BK / 4;    // W int8 bytes per stage, in floats
  constexpr int SS = 4 * 64;         // scale slots per stage (64 per wave, 32 used)
  constexpr int ST = SA + SW + SS;
  __shared__ __align__(1024) float L[kDmaStages * ST];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  size_t wsoff = 0;
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
      wsoff = g.seg[i].wsoff;
    }
  const int M = g.M, K = g.K, lda = g.lda;
  const int n0 = (static_cast<int>(blockIdx.x) - tile0) * BN;  // one row tile (M <= 32)
  const int nkt = K / BK;
  const int kb0 = static_cast<int>(blockIdx.y) * nkt / g.splits;
  const int kb1 = (static_cast<int>(blockIdx.y) + 1) * nkt / g.splits;

  // Per-lane source offsets (block 0): A row 8 wave + l / 8, its chunk
  // (l % 8) ^ dma_swz(row); W row 32 wave + l / 2, its half l % 2; the scale
  // of W row 32 wave + l % 32 (lanes 32..63 repeat lanes 0..31's).
  const int ra = 8 * wave + (lane >> 3);
  const unsigned int ga = static_cast<unsigned int>(
      (min(ra, M - 1) * lda + 4 * ((lane & 7) ^ dma_swz(ra))) * 4);
  const int rw = 32 * wave + (lane >> 1);
  const size_t gw = static_cast<size_t>(min(n0 + rw, N - 1)) * ldw + 16 * (lane & 1);
  const size_t gs = static_cast<size_t>(min(n0 + 32 * wave + (lane & 31), N - 1)) * ldw;
  auto request = [&](int kb, int st) {
    float* la = L + st * ST;
    __builtin_amdgcn_global_load_lds(
        (global_void_t*)(reinterpret_cast<const char*>(A) + static_cast<size_t>(kb) * BK * 4 + ga),
        (lds_void_t*)(la + 256 * wave), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(
        (global_void_t*)(static_cast<const char*>(W) + gw + static_cast<size_t>(kb) * BK),
        (lds_void_t*)(la + SA + 256 * wave), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(
        (global_void_t*)(S + ((gs + static_cast<size_t>(kb) * BK) >> gshift)),
        (lds_void_t*)(la + SA + SW + 64 * wave), 4, 0, 0);
  };
  const int g4 = lane >> 4, r16 = lane & 15;
  int oa[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) oa[j] = r16 * BK + 4 * ((2 * g4 + j) ^ dma_swz(r16));
  gf4 af[2][2][2], bf[2][2][2];  // [register buffer][block][16-byte group of k]
  auto operands = [&](int st, int p) {
    const float* la = L + st * ST;
    const unsigned char* lw = reinterpret_cast<const unsigned char*>(la + SA);
    const float* ls = la + SA + SW + 64 * wave;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int j = 0; j < 2; ++j) af[p][a][j] = *reinterpret_cast<const gf4*>(la + a * 16 * BK + oa[j]);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int row = 32 * wave + 16 * b + r16;
      const uint2 q = *reinterpret_cast<const uint2*>(lw + row * BK + 8 * g4);
      const float sc = ls[16 * b + r16];
      const int lo = static_cast<int>(q.x), hi = static_cast<int>(q.y);
      bf[p][b][0] = gf4{static_cast<float>((lo << 24) >> 24) * sc, static_cast<float>((lo << 16) >> 24) * sc,
                        static_cast<float>((lo << 8) >> 24) * sc, static_cast<float>(lo >> 24) * sc};
      bf[p][b][1] = gf4{static_cast<float>((hi << 24) >> 24) * sc, static_cast<float>((hi << 16) >> 24) * sc,
                        static_cast<float>((hi << 8) >> 24) * sc, static_cast<float>(hi >> 24) * sc};
    }
  };
  gf4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = gf4{0.f, 0.f, 0.f, 0.f};
  auto steps = [&](int p, int s0, int s1) {
#pragma unroll
    for (int s = s0; s < s1; ++s)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[p][a][s >> 2][s & 3], bf[p][b][s >> 2][s & 3],
                                                           acc[a][b], 0, 0, 0);
  };
  constexpr int kLoads = 3;  // load instructions per block and wave
  if (kb0 < kb1) {
    request(kb0, 0);
    request(min(kb0 + 1, kb1 - 1), 1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads) : "memory");
    __builtin_amdgcn_s_barrier();
    operands(0, 0);
    int st = 0;
    // As k_gemm_f32_dma: request block kt + 2, run 6 of the 8 k steps, wait
    // for block kt + 1 and every wave's reads, read its operands into the
    // other register buffer while the last 2 steps run.
    auto block = [&](int kt, int p) {
      const int sn = st == 0 ? 2 : st - 1;
      const int st1 = st == 2 ? 0 : st + 1;
      request(min(kt + 2, kb1 - 1), sn);
      steps(p, 0, 6);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(kLoads) : "memory");
      __builtin_amdgcn_s_barrier();
      operands(st1, p ^ 1);
      steps(p, 6, 8);
      st = st1;
    };
    int kt = kb0;
    for (; kt + 1 < kb1; kt += 2) {
      block(kt, 0);
      block(kt + 1, 1);
    }
    if (kt < kb1) block(kt, 0);
  }

  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * g.ws_split + wsoff : nullptr;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * a + 4 * g4 + r;
        const int n = n0 + 32 * wave + 16 * b + r16;
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

// ---------------------------------------------------------------------------
// Split-product GEMM (fp32 accuracy on the bf16 matrix cores).  Each fp32
// operand x is held as three bf16 planes x = x0 + x1 + x2 (x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1), round to nearest even;
// k_split3): 8 + 8 + 8 significand bits carry all 24 of x.  The product
// A W^T = sum over i, j of Ai Wj^T; the kernel forms the six terms with
// i + j <= 2, each a bf16 x bf16 product that fp32 holds exactly, accumulated
// in fp32 by v_mfma_f32_32x32x16_bf16.  The three terms left out (i + j >= 3)
// are each at most 2^-24 |a w| (|x1| <= 2^-8 |x|, |x2| <= 2^-16 |x|), the
// size of one fp32 rounding, so the result is as accurate as an fp32 GEMM
// (measured on the prefill shapes: max |error| / sum |a w| 3e-8 (split K) to
// 1.1e-7 (one K pass) against 1.3e-7 to 2.2e-7 for k_gemm_f32_dma).  bf16 MFMA
// runs at 16x the fp32 MFMA rate, six products at 2.7x.
//
// Workgroup tile 64 WMW x 128 with WMW = 2 (128 x 128, four waves, a 3-stage
// ring of 48 KB stages) or 4 (256 x 128, eight waves -- two per SIMD, so a
// wave waiting on its loads leaves the matrix core to the other -- a 2-stage
// ring of 72 KB; 25% fewer operand bytes per product).  A stage is refilled as
// soon as every wave holds its operands in registers (mid-block), so each
// block's loads are in flight for ST - 1 blocks of MFMA work; each wave 64 x 64 (2 x 2 blocks of 32 x 32;
// A operand: lane l holds A[l % 32][8 k-values], B operand W[l % 32][the
// same 8 k-values], k-values 8 (l / 32) .. + 7 of a 16-column step; result
// register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]).  The
// planes are stored in tiles of 16 rows x 32 columns, the three planes of a
// tile in 3 KB of consecutive memory (x6_tile_offset), so each 1 KB
// direct-to-LDS load instruction reads 1 KB of consecutive bytes (rows of 64
// B in row-major planes touch half of sixteen 128 B lines each: 7-11% slower
// on the Qwen3-4B and Qwen2.5-1.5B shapes).  K advances in blocks of 32
// columns: the six plane tiles of a block (A0 A1 A2 W0 W1 W2, rows of 64 B)
// land in LDS through the ring (144 KB either way: one workgroup per CU).
// A row holds four
// 16-byte chunks; chunk c of row r sits in slot c ^ x6_swz(r), so the 32
// lanes of a half wave (32 consecutive rows, one chunk each) read 32 distinct
// 16-byte slots of the 512 B bank period.  Each block runs as two 16-column steps of 24
// MFMAs (six products x four blocks); the second step's operands are read
// from LDS during the first step, the next block's first-step operands
// during the second (the reads are interleaved one per MFMA).
//
// Launch order is XCD-aware: workgroup b runs on XCD b % 8 (round-robin
// dispatch), so tile t = (b % 8) ceil(T / 8) + b / 8 gives each XCD a
// contiguous run of tiles whose M tiles share their W tile in its L2.
// Split-K as k_gemm_f32_dma (blockIdx.y = split, partials to ws, then
// k_gemm_reduce).  The launcher (gemm_run_x6) picks the tile, and may run a
// launch as whole rounds of tiles plus a split-K launch over the remaining
// columns of the last output, so that the partial last round is spread over
// every CU.
__device__ __forceinline__ int x6_swz(int r) { return (r >> 3) & 3; }

// Element (r, k) of plane p of an R x K matrix (K a multiple of 32) in the
// tiled plane format: tiles of 16 rows x 32 columns in row-tile-major order,
// each holding plane 0, 1, 2 (512 elements each, rows of 32).  A buffer holds
// ceil(R / 16) * 16 * K * 3 elements; rows past R in the last tile only feed
// outputs that are never stored.
__host__ __device__ __forceinline__ size_t x6_tile_offset(int r, int k, int p, int K) {
  return (static_cast<size_t>(r >> 4) * (K >> 5) + (k >> 5)) * 1536 + 512 * p + 32 * (r & 15) + (k & 31);
}

typedef __bf16 xbf8 __attribute__((ext_vector_type(8)));

// NPW = 1: W's planes 1 and 2 are all zero (W holds bf16 values exactly, as
// weights exported from bf16 checkpoints do); only plane 0 is loaded and the
// three terms Ai W0 are formed, in the order the six-term step forms them, so
// the result is the six-term one (the other three terms are exact zeros).
template <int WMW, int NPW>  // waves along M: 2 (128 x 128 tiles) or 4 (256 x 128); W planes
__global__ __launch_bounds__(128 * WMW) void k_gemm_x6(GemmX6Args x) {
  static_assert(NPW == 1 || NPW == 3, "weight planes");
  constexpr int BM = 64 * WMW, BN = 128, BK = 32, ST = WMW == 4 ? 2 : 3;
  constexpr int PA = BM * BK, PW = BN * BK;   // bf16 per plane tile (A, W)
  constexpr int SS = 3 * PA + NPW * PW;       // per stage
  constexpr int NW = 2 * WMW;                 // waves
  constexpr int NL = 3 * BM / 16 + NPW * BN / 16;  // 1 KB loads per stage
  constexpr int LPW = NL / NW;
  static_assert(LPW * NW == NL, "loads per wave");
  __shared__ __align__(1024) __bf16 L[ST * SS];
  const GemmArgs& g = x.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WMW, wn = wave / WMW;
  const int per = static_cast<int>(gridDim.x) >> 3;
  const int b = static_cast<int>(blockIdx.x);
  const int t = (b & 7) * per + (b >> 3);
  if (t >= x.tiles) return;
  int sidx = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < g.nseg && t >= g.seg[i].tile0) sidx = i;
  const char* W = static_cast<const char*>(x.p.W[0]);
  float* C = g.seg[0].C;
  const float* bias = g.seg[0].bias;
  int N = g.seg[0].N, ldc = g.seg[0].ldc, tile0 = 0;
  size_t wsoff = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i == sidx) {
      W = static_cast<const char*>(x.p.W[i]);
      C = g.seg[i].C;
      bias = g.seg[i].bias;
      N = g.seg[i].N;
      ldc = g.seg[i].ldc;
      tile0 = g.seg[i].tile0;
      wsoff = g.seg[i].wsoff;
    }
  const int M = g.M, K = g.K;
  const int local = t - tile0;
  const int tm = local % g.tiles_m, tn = local / g.tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nkt = K / BK;
  const int kb0 = static_cast<int>(blockIdx.y) * nkt / g.splits;
  const int kb1 = (static_cast<int>(blockIdx.y) + 1) * nkt / g.splits;
  const char* A = static_cast<const char*>(x.p.A);

  // Load instruction i of this wave fills 1 KB j = LPW wave + i of a stage:
  // plane (j / 8) % 3 of operand j < 24 ? A : W, rows 16 (j % 8) .. + 15 of
  // the workgroup tile (one 16-row tile of the plane format: 1 KB of
  // consecutive bytes per k block, the next k block 3 KB further on); lane l
  // fills slot l % 4 of row r = 16 (j % 8) + l / 4 with chunk
  // (l % 4) ^ x6_swz(r).  Row tiles past M or N read the last one (they only
  // feed outputs that are never stored).
  const char* src[LPW];
  int ldo[LPW];
  const int kbs = K / BK;
  const int lra = (M - 1) >> 4, lrw = (N - 1) >> 4;
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int j = LPW * wave + i;
    const bool isa = j < 3 * BM / 16;
    const int jj = isa ? j : j - 3 * BM / 16;
    const int rpp = isa ? BM / 16 : BN / 16;     // row tiles per plane
    const int pl = jj / rpp, tr = jj % rpp;
    const int c = (lane & 3) ^ x6_swz(16 * tr + (lane >> 2));
    const int rt = isa ? min((m0 >> 4) + tr, lra) : min((n0 >> 4) + tr, lrw);
    src[i] = (isa ? A : W) + (static_cast<size_t>(rt) * kbs * 1536 + 512 * pl) * 2 + 64 * (lane >> 2) + 16 * c;
    ldo[i] = isa ? pl * PA + 512 * tr : 3 * PA + pl * PW + 512 * tr;
  }
  auto request = [&](int kb, int st) {
    __bf16* base = L + st * SS;
#pragma unroll
    for (int i = 0; i < LPW; ++i)
      __builtin_amdgcn_global_load_lds((global_void_t*)(src[i] + static_cast<size_t>(kb) * 3072),
                                       (lds_void_t*)(base + ldo[i]), 16, 0, 0);
  };
  // Step s of a block: lane half h = l / 32 reads chunk 2 s + h of rows
  // 64 wm + 32 q + l % 32 (A planes) and 64 wn + 32 q + l % 32 (W planes).
  const int h = lane >> 5, r32 = lane & 31;
  int oa[2][2], ow[2][2];  // [block q][step s], bf16 offsets within a plane tile
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ra = 64 * wm + 32 * q + r32, rw = 64 * wn + 32 * q + r32;
      oa[q][s] = ra * BK + 8 * ((2 * s + h) ^ x6_swz(ra));
      ow[q][s] = rw * BK + 8 * ((2 * s + h) ^ x6_swz(rw));
    }
  xbf8 fa[2][3][2], fw[2][NPW][2];  // [register buffer][plane][block]
  auto operands = [&](int st, int s, int p) {
    const __bf16* base = L + st * SS;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        fa[p][pl][q] = *reinterpret_cast<const xbf8*>(base + pl * PA + oa[q][s]);
        if (pl < NPW) fw[p][pl][q] = *reinterpret_cast<const xbf8*>(base + 3 * PA + pl * PW + ow[q][s]);
      }
  };
  gf16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][c][r] = 0.f;
  // The six products of one step, smallest terms first (NPW = 1: the three
  // with W0, in the same relative order).
  auto step = [&](int p) {
    constexpr int NT = NPW == 3 ? 6 : 3;
    constexpr int PA[6] = {2, 1, 0, 1, 0, 0}, PW[6] = {0, 1, 2, 0, 1, 0};
    constexpr int PA1[3] = {2, 1, 0};
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[a][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[p][NPW == 3 ? PA[k] : PA1[k]][a],
                                                              fw[p][NPW == 3 ? PW[k] : 0][c], acc[a][c], 0,
                                                              0, 0);
  };
  // One LDS operand read (and, with loads, one direct-to-LDS request) after
  // each of the first (3 + NPW) 2 MFMAs of a step.
  constexpr int NRD = (3 + NPW) * 2, NMF = (NPW == 3 ? 6 : 3) * 4;
#define KL_X6_INTERLEAVE(loads)                                           \
  do {                                                                    \
    _Pragma("unroll") for (int i_ = 0; i_ < NRD; ++i_) {                  \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  \
      if (loads) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);       \
    }                                                                     \
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - NRD, 0);            \
  } while (0)
  if (kb0 < kb1) {
    // Prologue: blocks kb0 .. kb0 + ST - 1 requested (clamped to the last
    // block), block kb0 waited for.
#pragma unroll
    for (int s = 0; s < ST; ++s) request(min(kb0 + s, kb1 - 1), s);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((ST - 1) * LPW) : "memory");
    __builtin_amdgcn_s_barrier();
    operands(0, 0, 0);
    int st = 0;
    // Block kt in stage st, its first-step operands in register buffer 0:
    // read the second step's operands and run the first step; wait until
    // block kt + 1 has landed (ST - 2 later requests may still be in flight)
    // and every wave has read its operands of stage st, which is then free:
    // request block kt + ST into it, read block kt + 1's first step and run
    // the second step.  Each block's loads are thus in flight for ST - 1
    // blocks of MFMA work.  Requests past the last block load the last block
    // again into a stage nobody reads afterwards, so every wait is an exact
    // vmcnt; the loop ends with a full drain.
    for (int kt = kb0; kt < kb1; ++kt) {
      const int st1 = st == ST - 1 ? 0 : st + 1;
      __builtin_amdgcn_sched_barrier(0);
      operands(st, 1, 1);
      step(0);
      KL_X6_INTERLEAVE(false);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"((ST - 2) * LPW) : "memory");
      __builtin_amdgcn_s_barrier();
      request(min(kt + ST, kb1 - 1), st);
      operands(st1, 0, 0);
      step(1);
      KL_X6_INTERLEAVE(true);
      __builtin_amdgcn_sched_barrier(0);
      st = st1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
#undef KL_X6_INTERLEAVE
  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * g.ws_split + wsoff : nullptr;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 64 * wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
        const int n = n0 + 64 * wn + 32 * c + r32;
        if (m < M && n < N) {
          float v = acc[a][c][r];
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

// Stores the three bf16 planes of x[r][k .. k + 3] (k a multiple of 4): the
// tiled plane format of k_gemm_x6 (K columns), or k_gemm_q8s's lane order
// (q8s: r < 32).  The GEMM-input producers (row norm, SwiGLU) write through it.
typedef __bf16 xbf4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void planes_store4(bool q8s, __bf16* out, int r, int k, int K, gf4 v) {
  xbf4 x0, x1, x2;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x0[e] = static_cast<__bf16>(v[e]);
    const float r1 = v[e] - static_cast<float>(x0[e]);
    x1[e] = static_cast<__bf16>(r1);
    x2[e] = static_cast<__bf16>(r1 - static_cast<float>(x1[e]));
  }
  size_t off, ps;
  if (q8s) {
    const int j = k >> 5, kk = k & 31;
    off = ((static_cast<size_t>(j) * 3 * 2 + ((kk >> 3) & 1)) * 64 + (kk >> 4) * 32 + r) * 8 + (kk & 7);
    ps = 1024;
  } else {
    off = x6_tile_offset(r, k, 0, K);
    ps = 512;
  }
  *reinterpret_cast<xbf4*>(out + off) = x0;
  *reinterpret_cast<xbf4*>(out + off + ps) = x1;
  *reinterpret_cast<xbf4*>(out + off + 2 * ps) = x2;
}

// fp32 rows -> the three bf16 planes x0, x1, x2 of k_gemm_x6 in the tiled
// plane format (x6_tile_offset); eight values per thread.
// Whether planes 1 and 2 of a rows x K matrix in the tiled plane format hold
// any nonzero bit in rows < rows (tiles of 1536 bf16, row-tile-major: plane 0
// at 0, planes 1 and 2 at 512 .. 1535, rows of 32; the padding rows of the
// last row tile are never written): *flag |= 1 if so (a bf16-exact matrix
// splits into zero planes 1 and 2).
__global__ void k_x6_planes_nonzero(const unsigned* __restrict__ planes, int rows, int K, size_t tiles,
                                    unsigned* flag) {
  unsigned acc = 0;
  const size_t words = tiles * 512;  // 32-bit words of planes 1 and 2
  const int kt = K / 32;             // tiles per row tile
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < words;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t t = i / 512;
    const int w = static_cast<int>(i % 512);
    const int row = 16 * static_cast<int>(t / kt) + (w % 256) / 16;
    if (row < rows) acc |= planes[t * 768 + 256 + w];
  }
  if (acc) atomicOr(flag, 1u);
}

__global__ void k_split3(const float* __restrict__ x, int rows, int cols, int ldx,
                         __bf16* __restrict__ out) {
  const int c8 = cols / 8;
  const size_t total = static_cast<size_t>(rows) * c8;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int r = static_cast<int>(i / c8);
    const int c = static_cast<int>(i - static_cast<size_t>(r) * c8) * 8;
    const gf4* p = reinterpret_cast<const gf4*>(x + static_cast<size_t>(r) * ldx + c);
    const gf4 v0 = p[0], v1 = p[1];
    xbf8 x0, x1, x2;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = j < 4 ? v0[j] : v1[j - 4];
      x0[j] = static_cast<__bf16>(v);
      const float r1 = v - static_cast<float>(x0[j]);
      x1[j] = static_cast<__bf16>(r1);
      x2[j] = static_cast<__bf16>(r1 - static_cast<float>(x1[j]));
    }
    const size_t o = x6_tile_offset(r, c, 0, cols);
    *reinterpret_cast<xbf8*>(out + o) = x0;
    *reinterpret_cast<xbf8*>(out + o + 512) = x1;
    *reinterpret_cast<xbf8*>(out + o + 1024) = x2;
  }
}

// ---------------------------------------------------------------------------
// Short int8 prompts (at most 32 rows, group size 32 or 64): k_gemm_q8s.  The batched form of the reference int8 GEMV (float(q) * scale
// per weight, cuda/matmul_kernel.cu:73) computed as sum over groups g of
// scale[n][g] * sum_{k in g} a[k] q[n][k]: the activations as three bf16
// planes (k_split3's split, rows padded to 32), each int8 weight exactly a
// bf16, so the three products a_i q per multiply-add are exact in fp32 and
// accumulate in fp32 on v_mfma_f32_32x32x16_bf16, one group at a time, then
// scale into the output registers.  At 32 rows the launch is bound by the int8
// weight bytes (cfg 3: 6.9 GB for 32 tokens), so the weights are prepacked
// once (k_q8s_pack) in the order the lanes consume them: a 1 KB block per 32
// columns x 32 k holding, for lane l, the 16 bytes W[32 b + l % 32][32 j +
// 16 (l / 32) .. + 15], and the group scales as 128 B per (32 columns,
// group); every weight load is a whole 1 KB of consecutive bytes straight
// into registers, prefetched four groups ahead.  The
// activation planes use the same k order: plane p, k step s (8 values) of
// chunk j at element (((j * 3 + p) * 2 + s) * 64 + l) * 8 of the plane buffer,
// lane l holding A[l % 32][32 j + 16 (l / 32) + 8 s .. + 7] (k_q8s_split).  A
// workgroup of eight waves copies its split's activation planes (6 KB per
// chunk, at most kQ8sLdsChunks) into LDS once, behind one barrier, and each
// wave then streams the weights of its two 32-column blocks (32 x 64 of C):
// with the activations read from L2 by every wave instead, they were three
// times the weight bytes through each CU's load path and the kernel ran at
// 1.6-2.8 TB/s.  Split-K over whole groups (blockIdx.y) as k_gemm_f32_dma.
constexpr int kQ8sLdsChunks = 26;  // activation chunks a split may hold in LDS (156 KB)

__host__ __device__ inline size_t q8s_tile_bytes(int N, int K) {
  return static_cast<size_t>((N + 31) / 32) * (K / 32) * 1024;
}

typedef int gi4 __attribute__((ext_vector_type(4)));

// Byte e (sign-extended) of w -> float: one SDWA conversion (the compiler
// shifts the odd bytes first otherwise).
template <int E>
__device__ __forceinline__ float q8s_byte(int w) {
  float f;
  if constexpr (E == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(f) : "v"(w));
  else if constexpr (E == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(f) : "v"(w));
  else if constexpr (E == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(f) : "v"(w));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(f) : "v"(w));
  return f;
}

// Eight int8 (two 32-bit words) -> eight bf16 (exact).
__device__ __forceinline__ xbf8 q8s_bf16(int lo, int hi) {
  xbf8 r;
  r[0] = static_cast<__bf16>(q8s_byte<0>(lo));
  r[1] = static_cast<__bf16>(q8s_byte<1>(lo));
  r[2] = static_cast<__bf16>(q8s_byte<2>(lo));
  r[3] = static_cast<__bf16>(q8s_byte<3>(lo));
  r[4] = static_cast<__bf16>(q8s_byte<0>(hi));
  r[5] = static_cast<__bf16>(q8s_byte<1>(hi));
  r[6] = static_cast<__bf16>(q8s_byte<2>(hi));
  r[7] = static_cast<__bf16>(q8s_byte<3>(hi));
  return r;
}

template <int CPG>  // 32-column chunks per scale group (group size 32 CPG)
__global__ __launch_bounds__(512, 1) void k_gemm_q8s(GemmQ8sArgs g) {
  static_assert(CPG == 1 || CPG == 2, "group size 32 or 64");
  constexpr int GD = 4;  // groups in flight
  __shared__ __align__(1024) char Al[kQ8sLdsChunks * 6144];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bx = static_cast<int>(blockIdx.x);
  int sidx = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i < g.nseg && bx >= g.seg[i].wg0) sidx = i;
  const char* P = static_cast<const char*>(g.seg[0].P);
  float* C = g.seg[0].C;
  const float* bias = g.seg[0].bias;
  int N = g.seg[0].N, ldc = g.seg[0].ldc, wg0 = 0;
  size_t wsoff = 0;
#pragma unroll
  for (int i = 1; i < kGemmMaxSeg; ++i)
    if (i == sidx) {
      P = static_cast<const char*>(g.seg[i].P);
      C = g.seg[i].C;
      bias = g.seg[i].bias;
      N = g.seg[i].N;
      ldc = g.seg[i].ldc;
      wg0 = g.seg[i].wg0;
      wsoff = g.seg[i].wsoff;
    }
  const int K = g.K, nc = K / 32, ng = K / (32 * CPG);
  const int gb = static_cast<int>(blockIdx.y) * ng / g.splits;
  const int ge = (static_cast<int>(blockIdx.y) + 1) * ng / g.splits;
  // The split's activation planes (6 KB per chunk, consecutive) into LDS,
  // spread over the waves; every wave then streams only its own weights.
  {
    const char* src = static_cast<const char*>(g.A) + static_cast<size_t>(gb) * CPG * 6144 + 16 * lane;
    const int n1k = (ge - gb) * CPG * 6;
    for (int i = wave; i < n1k; i += 8)
      __builtin_amdgcn_global_load_lds((global_void_t*)(src + static_cast<size_t>(i) * 1024),
                                       (lds_void_t*)(Al + 1024 * i), 16, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
  const int nb = (N + 31) / 32;
  const int b0 = 16 * (bx - wg0) + 2 * wave;
  if (b0 >= nb || gb >= ge) return;  // past the last barrier: waves leave on their own
  const int b1 = min(b0 + 1, nb - 1);
  const char* w0 = P + static_cast<size_t>(b0) * nc * 1024 + 16 * lane;
  const char* w1 = P + static_cast<size_t>(b1) * nc * 1024 + 16 * lane;
  const float* S = reinterpret_cast<const float*>(P + q8s_tile_bytes(N, K));
  const float* s0p = S + static_cast<size_t>(b0) * ng * 32 + (lane & 31);
  const float* s1p = S + static_cast<size_t>(b1) * ng * 32 + (lane & 31);
  const char* Ap = Al + 16 * lane;
  gf16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc0[r] = acc1[r] = 0.f;
  gi4 wq[GD][CPG][2];  // raw int8 fragments of the groups in flight
  float sc[GD][2];
  xbf8 qb[2][CPG][2][2];  // bf16 weights: [buffer][chunk][block][k step]
  // Group grp (clamped to the split's last) into ring slot u: its chunks'
  // weight fragments (1 KB per block and chunk) and scales.
  auto load = [&](int grp, int u) {
    const int gg = min(grp, ge - 1);
#pragma unroll
    for (int c = 0; c < CPG; ++c) {
      const size_t j = static_cast<size_t>(gg) * CPG + c;
      wq[u][c][0] = __builtin_nontemporal_load(reinterpret_cast<const gi4*>(w0 + j * 1024));
      wq[u][c][1] = __builtin_nontemporal_load(reinterpret_cast<const gi4*>(w1 + j * 1024));
    }
    sc[u][0] = s0p[static_cast<size_t>(gg) * 32];
    sc[u][1] = s1p[static_cast<size_t>(gg) * 32];
  };
  auto convert = [&](int u, int v) {
#pragma unroll
    for (int c = 0; c < CPG; ++c)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int st = 0; st < 2; ++st) qb[v][c][b][st] = q8s_bf16(wq[u][c][b][2 * st], wq[u][c][b][2 * st + 1]);
  };
  // Group grp (ring slot u, bf16 weights in buffer v): its activation
  // fragments from LDS, then the MFMAs, with the next group (slot un) converted
  // into buffer v ^ 1 in their shadow (a few VALU instructions after each
  // MFMA: converting first and multiplying after left the VALU and the matrix
  // core taking turns), then the group's sums scaled into acc.
  auto group = [&](int grp, int u, int v, int un) {
    xbf8 a[CPG][3][2];
#pragma unroll
    for (int c = 0; c < CPG; ++c) {
      const int jl = (grp - gb) * CPG + c;
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int st = 0; st < 2; ++st)
          a[c][p][st] = *reinterpret_cast<const xbf8*>(Ap + ((jl * 3 + p) * 2 + st) * 1024);
    }
    gf16 t[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) t[0][r] = t[1][r] = 0.f;
#pragma unroll
    for (int c = 0; c < CPG; ++c)
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int p = 2; p >= 0; --p)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            t[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][p][st], qb[v][c][b][st], t[b], 0, 0, 0);
    convert(un, v ^ 1);
    // 12 CPG MFMAs; 12 CPG conversions of 4 values (2 VALU each) and 2 CPG LDS reads per MFMA slot
#pragma unroll
    for (int i = 0; i < 12 * CPG; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc0[r] += sc[u][0] * t[0][r];
      acc1[r] += sc[u][1] * t[1][r];
    }
  };
#pragma unroll
  for (int u = 0; u < GD; ++u) load(gb + u, u);
  convert(0, 0);
  int grp = gb;
  // Ring slot of group gb + i is i % GD and its bf16 buffer i % 2 (GD even):
  // an unroll of GD keeps both compile-time.
  for (; grp + GD <= ge; grp += GD) {
#pragma unroll
    for (int i = 0; i < GD; ++i) {
      group(grp + i, i, i & 1, (i + 1) % GD);
      load(grp + i + GD, i);
    }
  }
#pragma unroll
  for (int i = 0; i < GD; ++i)
    if (grp + i < ge) group(grp + i, i, i & 1, (i + 1) % GD);
  const int h = lane >> 5;
  float* wsp = g.splits > 1 ? g.ws + static_cast<size_t>(blockIdx.y) * g.ws_split + wsoff : nullptr;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int n = 32 * (q ? b0 + 1 : b0) + (lane & 31);
    if (n >= N) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 8 * (r >> 2) + 4 * h + (r & 3);
      if (m < g.M) {
        float v = q ? acc1[r] : acc0[r];
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
}

// int8 weights [N x K] (row-major, scales[(n K + k) >> gshift]) -> the packed
// order of k_gemm_q8s: one thread per 16-byte lane fragment, then the scales.
// Rows past N are zero.
__global__ void k_q8s_pack(const int8_t* __restrict__ q, const float* __restrict__ sc, int N, int K,
                           int gshift, char* __restrict__ out) {
  const int nb = (N + 31) / 32, nc = K / 32, ng = K >> gshift;
  const size_t frags = static_cast<size_t>(nb) * nc * 64;
  const size_t scales = static_cast<size_t>(nb) * ng * 32;
  float* so = reinterpret_cast<float*>(out + q8s_tile_bytes(N, K));
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < frags + scales;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    if (i < frags) {
      const int l = static_cast<int>(i & 63);
      const size_t bj = i >> 6;
      const int b = static_cast<int>(bj / nc), j = static_cast<int>(bj % nc);
      const int n = 32 * b + (l & 31), k = 32 * j + 16 * (l >> 5);
      gi4 v = {0, 0, 0, 0};
      if (n < N) v = *reinterpret_cast<const gi4*>(q + static_cast<size_t>(n) * K + k);
      *reinterpret_cast<gi4*>(out + 16 * i) = v;
    } else {
      const size_t t = i - frags;
      const int nn = static_cast<int>(t & 31);
      const size_t bg = t >> 5;
      const int b = static_cast<int>(bg / ng), grp = static_cast<int>(bg % ng);
      const int n = 32 * b + nn;
      so[t] = n < N ? sc[(static_cast<size_t>(n) * K >> gshift) + grp] : 0.f;
    }
  }
}

// Activation rows (at most 32, row stride ldx) -> the three bf16 planes of
// k_gemm_q8s in its lane order (rows past M are zero).
__global__ void k_q8s_split(const float* __restrict__ x, int M, int K, int ldx, __bf16* __restrict__ out) {
  const size_t total = static_cast<size_t>(K / 32) * 2 * 64;  // (chunk, step, lane)
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int l = static_cast<int>(i & 63);
    const int st = static_cast<int>((i >> 6) & 1);
    const int j = static_cast<int>(i >> 7);
    const int m = l & 31, k = 32 * j + 16 * (l >> 5) + 8 * st;
    gf4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
    if (m < M) {
      const gf4* src = reinterpret_cast<const gf4*>(x + static_cast<size_t>(m) * ldx + k);
      v0 = src[0];
      v1 = src[1];
    }
    xbf8 x0, x1, x2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = e < 4 ? v0[e] : v1[e - 4];
      x0[e] = static_cast<__bf16>(v);
      const float r1 = v - static_cast<float>(x0[e]);
      x1[e] = static_cast<__bf16>(r1);
      x2[e] = static_cast<__bf16>(r1 - static_cast<float>(x1[e]));
    }
    const size_t base = ((static_cast<size_t>(j) * 3) * 2 + st) * 512 + 8 * l;
    *reinterpret_cast<xbf8*>(out + base) = x0;
    *reinterpret_cast<xbf8*>(out + base + 1024) = x1;
    *reinterpret_cast<xbf8*>(out + base + 2048) = x2;
  }
}

// C_s = sum of the split partials in split order (+ bias_s) (+ C_s), over
// every output s of the launch: element i of a split's slab belongs to the
// output whose [M][N_s] block (at seg[s].wsoff) holds it.
// p[0] + p[stride] + ... + p[(splits - 1) stride], added in that order (the
// bits of a plain loop), with the loads issued eight at a time ahead of their
// adds: a loop that waits for each partial before requesting the next pays one
// memory latency per split.
template <class T>
__device__ __forceinline__ T split_sum(const T* p, size_t stride, int splits) {
  T v = p[0];
  for (int z = 1; z < splits; z += 8) {
    T t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = p[static_cast<size_t>(min(z + j, splits - 1)) * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (z + j < splits) v += t[j];
  }
  return v;
}

__global__ void k_gemm_reduce(GemmArgs g) {
  const size_t total = g.ws_split;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    float* C = g.seg[0].C;
    const float* bias = g.seg[0].bias;
    int N = g.seg[0].N, ldc = g.seg[0].ldc;
    size_t off = 0;
#pragma unroll
    for (int k = 1; k < kGemmMaxSeg; ++k)
      if (k < g.nseg && i >= g.seg[k].wsoff) {
        C = g.seg[k].C;
        bias = g.seg[k].bias;
        N = g.seg[k].N;
        ldc = g.seg[k].ldc;
        off = g.seg[k].wsoff;
      }
    float v = split_sum(g.ws + i, total, g.splits);
    const size_t local = i - off;
    const int m = static_cast<int>(local / N), n = static_cast<int>(local - static_cast<size_t>(m) * N);
    if (bias) v += bias[n];
    float* cp = C + static_cast<size_t>(m) * ldc + n;
    if (g.accumulate) v = *cp + v;
    *cp = v;
  }
}

}  // namespace kl
