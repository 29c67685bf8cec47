// Causal attention of a batch of prompt positions for the batched prefill:
// the semantics of kernels/cpu/mha_kernel.cpp:5-61 (per head h, kv head
// h / kv_mul: softmax_t((q_h . K_t) / sqrt(hd)) . V_t over t <= position) for
// query positions pos0 .. pos0 + n - 1 at once, reading K and V rows 0 ..
// pos0 + n - 1 of one layer's caches ([seq_len][kv_dim]).
//
// One workgroup (256 threads) owns 64 query rows of one head and walks the
// key positions in blocks of 64 through LDS with an online softmax: thread
// (rg, cg) = (tid / 16, tid % 16) scores rows 4 rg .. 4 rg + 3 against keys
// 4 cg .. 4 cg + 3 of the block, the 16 threads of a row group combine the
// row maxima and sums with lane shuffles, and the same thread accumulates
// output columns cg * HD / 16 .. of its 4 rows.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>

namespace kl {

typedef float pf4 __attribute__((ext_vector_type(4)));

constexpr int kPrefillQB = 64;  // query rows per workgroup
constexpr int kPrefillKB = 64;  // key positions per block

__host__ __device__ constexpr size_t attn_prefill_lds_bytes(int hd) {
  return (static_cast<size_t>(kPrefillQB + 2 * kPrefillKB) * (hd + 4) +
          static_cast<size_t>(kPrefillQB) * (kPrefillKB + 4)) * sizeof(float);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ q, int ldq,
                                                      const float* __restrict__ kc,
                                                      const float* __restrict__ vc, int kv_dim,
                                                      int kv_mul, float* __restrict__ out, int ldo,
                                                      int pos0, int n, float scale) {
  constexpr int QB = kPrefillQB, KB = kPrefillKB, LD = HD + 4, LP = KB + 4, DPT = HD / 16;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;
  float* Ks = Qs + QB * LD;
  float* Vs = Ks + KB * LD;
  float* Ps = Vs + KB * LD;
  const int h = blockIdx.y, g = h / kv_mul;
  const int p0 = blockIdx.x * QB;
  const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;

  for (int i = tid; i < QB * HD / 4; i += 256) {
    const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
    const int p = p0 + r;
    const pf4 v = p < n ? *reinterpret_cast<const pf4*>(q + static_cast<size_t>(p) * ldq + h * HD + c)
                        : pf4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<pf4*>(Qs + r * LD + c) = v;
  }
  float m[4], l[4], o[4][DPT];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    m[a] = -INFINITY;
    l[a] = 0.f;
#pragma unroll
    for (int c = 0; c < DPT; ++c) o[a][c] = 0.f;
  }
  const int rows = n - p0 < QB ? n - p0 : QB;
  const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
  for (int j0 = 0; j0 <= last; j0 += KB) {
    __syncthreads();  // the previous block's K, V and P are consumed
    for (int i = tid; i < KB * HD / 4; i += 256) {
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const int j = j0 + r;
      const size_t off = static_cast<size_t>(j <= last ? j : 0) * kv_dim + g * HD + c;
      const pf4 kv = *reinterpret_cast<const pf4*>(kc + off);
      const pf4 vv = *reinterpret_cast<const pf4*>(vc + off);
      *reinterpret_cast<pf4*>(Ks + r * LD + c) = j <= last ? kv : pf4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<pf4*>(Vs + r * LD + c) = j <= last ? vv : pf4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    float s[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) s[a][b] = 0.f;
    for (int d = 0; d < HD; d += 4) {
      pf4 qv[4], kv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) qv[a] = *reinterpret_cast<const pf4*>(Qs + (4 * rg + a) * LD + d);
#pragma unroll
      for (int b = 0; b < 4; ++b) kv[b] = *reinterpret_cast<const pf4*>(Ks + (4 * cg + b) * LD + d);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          s[a][b] += qv[a].x * kv[b].x + qv[a].y * kv[b].y + qv[a].z * kv[b].z + qv[a].w * kv[b].w;
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int qpos = pos0 + p0 + 4 * rg + a;
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int kpos = j0 + 4 * cg + b;
        s[a][b] = kpos <= qpos ? s[a][b] * scale : -INFINITY;
        mx = fmaxf(mx, s[a][b]);
      }
#pragma unroll
      for (int w = 1; w < 16; w <<= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 16));
      const float mn = fmaxf(m[a], mx);
      // Key 0 is in the first block for every row, so mn is finite from then on.
      const float alpha = m[a] == -INFINITY ? 0.f : expf(m[a] - mn);
      float rs = 0.f;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float pv = s[a][b] == -INFINITY ? 0.f : expf(s[a][b] - mn);
        Ps[(4 * rg + a) * LP + 4 * cg + b] = pv;
        rs += pv;
      }
#pragma unroll
      for (int w = 1; w < 16; w <<= 1) rs += __shfl_xor(rs, w, 16);
      l[a] = l[a] * alpha + rs;
      m[a] = mn;
#pragma unroll
      for (int c = 0; c < DPT; ++c) o[a][c] *= alpha;
    }
    __syncthreads();
    const int jn = last - j0 + 1 < KB ? last - j0 + 1 : KB;
    for (int j = 0; j < jn; ++j) {
      float pj[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) pj[a] = Ps[(4 * rg + a) * LP + j];
      const float* vr = Vs + j * LD + cg * DPT;
#pragma unroll
      for (int c = 0; c < DPT; ++c) {
        const float v = vr[c];
#pragma unroll
        for (int a = 0; a < 4; ++a) o[a][c] += pj[a] * v;
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int p = p0 + 4 * rg + a;
    if (p < n) {
      float* op = out + static_cast<size_t>(p) * ldo + h * HD + cg * DPT;
#pragma unroll
      for (int c = 0; c < DPT; ++c) op[c] = o[a][c] / l[a];
    }
  }
}

// The same attention on the matrix cores (head sizes 64 and 128):
// flash-attention over key blocks of 64 with v_mfma_f32_32x32x2f32 (lane l
// supplies A[l % 32][k = l / 32] and B[k = l / 32][l % 32]; result register r
// of lane l is D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]).  Four waves per
// 64 query rows of one head: wave (wm, wn) = (w % 2, w / 2) computes the
// scores of rows 32 wm .. against keys 32 wn .. of the block (S = Q K^T, k
// running over d), and the output of rows 32 wm .. for columns wn HD / 2 ..
// (O += P V, k running over the 64 keys).  In both products lane half h takes
// the k indices of its half of the range in order: a lane's Q row slice stays
// in registers and its K and P operands are contiguous runs of a row in LDS;
// the V operand of step s is one float of key row 32 h + s, read by the 32
// lanes of a half as consecutive floats.  Only the row maxima cross waves
// (through LDS); each wave keeps the partial row sums of its key half,
// combined at the end.
// Maximum / sum over the 32 lanes of each half wave, in every lane: DPP
// within each 16-lane row (quad permutes and mirrors), then one exchange
// between the two rows of the half.
template <int CTRL>
__device__ __forceinline__ float pf_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float half_max(float v) {
  v = fmaxf(v, pf_dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, pf_dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, pf_dpp<0x141>(v));  // row_half_mirror
  v = fmaxf(v, pf_dpp<0x140>(v));  // row_mirror
  return fmaxf(v, __shfl_xor(v, 16, 32));
}
__device__ __forceinline__ float half_sum(float v) {
  v += pf_dpp<0xB1>(v);
  v += pf_dpp<0x4E>(v);
  v += pf_dpp<0x141>(v);
  v += pf_dpp<0x140>(v);
  return v + __shfl_xor(v, 16, 32);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill_mfma(const float* __restrict__ q, int ldq,
                                                           const float* __restrict__ kc,
                                                           const float* __restrict__ vc,
                                                           int kv_dim, int kv_mul,
                                                           float* __restrict__ out, int ldo,
                                                           int pos0, int n, float scale) {
  static_assert(HD == 64 || HD == 128, "head size");
  typedef float f16v __attribute__((ext_vector_type(16)));
  constexpr int QB = kPrefillQB, KB = kPrefillKB;
  constexpr int LDK = HD + 4;  // K and V row (floats)
  constexpr int LDP = KB + 4;  // P row
  constexpr int HH = HD / 2;   // d per lane half (scores) and columns per wave (output)
  constexpr int OT = HH / 32;  // 32 x 32 output tiles per wave
  extern __shared__ __align__(16) float sm[];
  float* Ks = sm;                 // [KB][LDK]
  float* Vs = Ks + KB * LDK;      // [KB][LDK]
  float* Ps = Vs + KB * LDK;      // [QB][LDP]
  float* rmax = Ps + QB * LDP;    // [2][QB] per key half
  float* rsum = rmax + 2 * QB;    // [2][QB]
  const int h = blockIdx.y, g = h / kv_mul;
  const int p0 = blockIdx.x * QB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1, hl = lane >> 5, li = lane & 31;

  // This lane's Q slice: row 32 wm + li, d in [HH hl, HH hl + HH).
  pf4 qr[HH / 4];
  {
    const int p = p0 + 32 * wm + li;
    const float* qp = q + static_cast<size_t>(p < n ? p : 0) * ldq + h * HD + HH * hl;
#pragma unroll
    for (int j = 0; j < HH / 4; ++j)
      qr[j] = p < n ? *reinterpret_cast<const pf4*>(qp + 4 * j) : pf4{0.f, 0.f, 0.f, 0.f};
  }
  // Rows of this lane's accumulator registers: 32 wm + 8 (r / 4) + 4 hl + r % 4.
  float m[16], lsum[16];
  f16v o[OT];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    m[r] = -INFINITY;
    lsum[r] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < OT; ++t) o[t] = f16v{};
  const int rows = n - p0 < QB ? n - p0 : QB;
  const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
  const int qbase = pos0 + p0 + 32 * wm + 4 * hl;
  // K and V of the next key block are loaded into registers while the current
  // block is multiplied.
  constexpr int NL = KB * HD / 4 / 256;  // float4s of K (and of V) per thread
  pf4 kpre[NL], vpre[NL];
  auto kvload = [&](int j0) {
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = tid + 256 * t;
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const int j = j0 + r;
      const size_t off = static_cast<size_t>(j <= last ? j : 0) * kv_dim + g * HD + c;
      kpre[t] = *reinterpret_cast<const pf4*>(kc + off);
      vpre[t] = *reinterpret_cast<const pf4*>(vc + off);
    }
  };
  kvload(0);
  for (int j0 = 0; j0 <= last; j0 += KB) {
    __syncthreads();  // the previous block's K, V and P are consumed
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = tid + 256 * t;
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const bool live = j0 + r <= last;
      *reinterpret_cast<pf4*>(Ks + r * LDK + c) = live ? kpre[t] : pf4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<pf4*>(Vs + r * LDK + c) = live ? vpre[t] : pf4{0.f, 0.f, 0.f, 0.f};
    }
    if (j0 + KB <= last) kvload(j0 + KB);
    __syncthreads();
    // S = Q K^T for rows 32 wm .., keys 32 wn .. of the block.
    f16v sacc = f16v{};
    {
      const float* kp = Ks + (32 * wn + li) * LDK + HH * hl;
#pragma unroll
      for (int j = 0; j < HH / 4; ++j) {
        const pf4 kv = *reinterpret_cast<const pf4*>(kp + 4 * j);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].x, kv.x, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].y, kv.y, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].z, kv.z, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].w, kv.w, sacc, 0, 0, 0);
      }
    }
    // Scale, causal mask, and the row maxima over this wave's 32 keys.
    const int kpos = j0 + 32 * wn + li;
    float sv[16], mx[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qpos = qbase + 8 * (r >> 2) + (r & 3);
      sv[r] = kpos <= qpos ? sacc[r] * scale : -INFINITY;
      mx[r] = half_max(sv[r]);
    }
    if (li == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax[wn * QB + 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3)] = mx[r];
    }
    __syncthreads();
    float alpha[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3);
      const float mn = fmaxf(m[r], fmaxf(mx[r], rmax[(1 - wn) * QB + row]));
      // A row whose keys so far are all masked (only in a part after the
      // first) keeps m = -inf, p = 0 and o = 0.
      alpha[r] = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
      m[r] = mn;
      const float pv = sv[r] == -INFINITY ? 0.f : expf(sv[r] - mn);
      Ps[row * LDP + 32 * wn + li] = pv;
      lsum[r] = lsum[r] * alpha[r] + half_sum(pv);
    }
    __syncthreads();
    // O = O alpha + P V for rows 32 wm .., columns wn HH + 32 t ...
#pragma unroll
    for (int t = 0; t < OT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha[r];
    {
      const float* pp = Ps + (32 * wm + li) * LDP + 32 * hl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const pf4 pv = *reinterpret_cast<const pf4*>(pp + 4 * j);
#pragma unroll
        for (int t = 0; t < OT; ++t) {
          const float* vp = Vs + (32 * hl + 4 * j) * LDK + wn * HH + 32 * t + li;
          o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.x, vp[0], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.y, vp[LDK], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.z, vp[2 * LDK], o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.w, vp[3 * LDK], o[t], 0, 0, 0);
        }
      }
    }
  }
  // Row sums: this wave's key half plus the other's.
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) rsum[wn * QB + 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3)] = lsum[r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3);
    const int p = p0 + row;
    if (p < n) {
      const float l = lsum[r] + rsum[(1 - wn) * QB + row];
      float* op = out + static_cast<size_t>(p) * ldo + h * HD + wn * HH + li;
#pragma unroll
      for (int t = 0; t < OT; ++t) op[32 * t] = o[t][r] / l;
    }
  }
}

// Head size 128 with eight waves per workgroup, two per SIMD, so that one
// wave's LDS reads, softmax and barriers overlap the other's matrix-core work
// (the four-wave kernel above leaves one wave per SIMD: 311 VGPRs + AGPRs).
// Key blocks of 128; wave (wm, wn) = (w % 2, w / 2) computes the scores of
// rows 32 wm .. against keys 32 wn .. of the block (k over d; its Q row slice
// in registers as above) and the output of rows 32 wm .. for columns 32 wn ..
// (k over the block's 128 keys: lane half h takes keys 64 h .. 64 h + 63).
// K and V of a block share one LDS buffer: K while the scores are computed,
// then V, loaded into registers during the scores.  The next block's K is
// loaded into registers during the current block.  Row maxima and sums cross
// the four key quarters through LDS and are combined in a fixed order.
//
// Key-range split (nparts > 1, blockIdx.z = part): where a chunk of rows far
// into the context gives fewer (row block, head) workgroups than the device
// has CUs, each one's key blocks are cut into nparts contiguous ranges, one
// workgroup each; a workgroup then writes its rows' unnormalised output with
// their running maximum and sum to `part` (an empty range writes max -inf,
// sum 0), and k_attn_prefill_merge8 combines the parts in order.
constexpr int kPrefillKB8 = 128;

// One partial record per query row: HD output floats, then max and sum,
// padded to a multiple of 4 floats so that every record (and every float4
// column group the merge reads) starts 16-byte aligned.
__host__ __device__ constexpr size_t attn_prefill_part_floats(int hd) { return hd + 4; }

template <int HD>
__global__ __launch_bounds__(512) void k_attn_prefill_mfma8(const float* __restrict__ q, int ldq,
                                                            const float* __restrict__ kc,
                                                            const float* __restrict__ vc,
                                                            int kv_dim, int kv_mul,
                                                            float* __restrict__ out, int ldo,
                                                            int pos0, int n, float scale,
                                                            int nparts, float* __restrict__ part) {
  static_assert(HD == 128, "head size");
  typedef float f16v __attribute__((ext_vector_type(16)));
  constexpr int QB = kPrefillQB, KB = kPrefillKB8;
  constexpr int LDK = HD + 4;  // K / V row (floats)
  constexpr int LDP = KB + 4;  // P row
  constexpr int HH = HD / 2;   // d per lane half (scores)
  constexpr int KH = KB / 2;   // keys per lane half (output)
  constexpr int NT = 512;
  extern __shared__ __align__(16) float sm[];
  float* KVs = sm;              // [KB][LDK]: the block's K, then its V
  float* Ps = KVs + KB * LDK;   // [QB][LDP]
  float* rmax = Ps + QB * LDP;  // [4][QB] per key quarter
  float* rsum = rmax + 4 * QB;  // [4][QB]
  const int h = blockIdx.y, g = h / kv_mul;
  const int p0 = blockIdx.x * QB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1, hl = lane >> 5, li = lane & 31;

  pf4 qr[HH / 4];  // Q row 32 wm + li, d in [HH hl, HH hl + HH)
  {
    const int p = p0 + 32 * wm + li;
    const float* qp = q + static_cast<size_t>(p < n ? p : 0) * ldq + h * HD + HH * hl;
#pragma unroll
    for (int j = 0; j < HH / 4; ++j)
      qr[j] = p < n ? *reinterpret_cast<const pf4*>(qp + 4 * j) : pf4{0.f, 0.f, 0.f, 0.f};
  }
  // Rows of this lane's accumulator registers: 32 wm + 8 (r / 4) + 4 hl + r % 4.
  float m[16], lsum[16];
  f16v o = f16v{};
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    m[r] = -INFINITY;
    lsum[r] = 0.f;
  }
  const int rows = n - p0 < QB ? n - p0 : QB;
  const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
  const int qbase = pos0 + p0 + 32 * wm + 4 * hl;
  // This workgroup's key blocks [kb0, kb1): all of them, or part blockIdx.z.
  const int nkb = last / KB + 1;
  const int kb0 = static_cast<int>(blockIdx.z) * nkb / nparts;
  const int kb1 = (static_cast<int>(blockIdx.z) + 1) * nkb / nparts;
  constexpr int NL = KB * HD / 4 / NT;  // float4s of K (and of V) per thread
  pf4 kpre[NL], vcur[NL];
  auto load = [&](const float* base, int j0, pf4* dst) {
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = tid + NT * t;
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const int j = j0 + r;
      dst[t] = *reinterpret_cast<const pf4*>(base + static_cast<size_t>(j <= last ? j : 0) * kv_dim +
                                             g * HD + c);
    }
  };
  auto stage = [&](int j0, const pf4* src) {  // rows past `last` as zeros
#pragma unroll
    for (int t = 0; t < NL; ++t) {
      const int i = tid + NT * t;
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      *reinterpret_cast<pf4*>(KVs + r * LDK + c) = j0 + r <= last ? src[t] : pf4{0.f, 0.f, 0.f, 0.f};
    }
  };
  const int jend = kb1 * KB;  // one past the last key of this workgroup's range
  if (kb0 < kb1) load(kc, kb0 * KB, kpre);
  for (int j0 = kb0 * KB; j0 < jend; j0 += KB) {
    __syncthreads();  // the previous block's V and P are consumed
    stage(j0, kpre);
    load(vc, j0, vcur);                          // this block's V, used after the scores
    if (j0 + KB < jend) load(kc, j0 + KB, kpre);  // the next block's K
    __syncthreads();
    // S = Q K^T for rows 32 wm .., keys 32 wn .. of the block.
    f16v sacc = f16v{};
    {
      const float* kp = KVs + (32 * wn + li) * LDK + HH * hl;
#pragma unroll
      for (int j = 0; j < HH / 4; ++j) {
        const pf4 kv = *reinterpret_cast<const pf4*>(kp + 4 * j);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].x, kv.x, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].y, kv.y, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].z, kv.z, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qr[j].w, kv.w, sacc, 0, 0, 0);
      }
    }
    // Scale, causal mask, and the row maxima over this wave's 32 keys.
    const int kpos = j0 + 32 * wn + li;
    float sv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qpos = qbase + 8 * (r >> 2) + (r & 3);
      sv[r] = kpos <= qpos ? sacc[r] * scale : -INFINITY;
      const float mx = half_max(sv[r]);
      if (li == 0) rmax[wn * QB + 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3)] = mx;
    }
    __syncthreads();  // every wave's scores are done (K is dead) and its maxima visible
    stage(j0, vcur);
    float alpha[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3);
      const float mn = fmaxf(fmaxf(m[r], fmaxf(rmax[row], rmax[QB + row])),
                             fmaxf(rmax[2 * QB + row], rmax[3 * QB + row]));
      // Key 0 is in the first block for every row, so mn is finite from then on.
      alpha[r] = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
      m[r] = mn;
      const float pv = sv[r] == -INFINITY ? 0.f : expf(sv[r] - mn);
      Ps[row * LDP + 32 * wn + li] = pv;
      lsum[r] = lsum[r] * alpha[r] + half_sum(pv);
    }
    __syncthreads();  // P and V are in LDS
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] *= alpha[r];
    // O = O alpha + P V for rows 32 wm .., columns 32 wn ...
    {
      const float* pp = Ps + (32 * wm + li) * LDP + KH * hl;
      const float* vb = KVs + KH * hl * LDK + 32 * wn + li;
#pragma unroll
      for (int j = 0; j < KH / 4; ++j) {
        const pf4 pv = *reinterpret_cast<const pf4*>(pp + 4 * j);
        const float* vp = vb + 4 * j * LDK;
        o = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.x, vp[0], o, 0, 0, 0);
        o = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.y, vp[LDK], o, 0, 0, 0);
        o = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.z, vp[2 * LDK], o, 0, 0, 0);
        o = __builtin_amdgcn_mfma_f32_32x32x2f32(pv.w, vp[3 * LDK], o, 0, 0, 0);
      }
    }
  }
  // Row sums: the four key quarters, in a fixed order.
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) rsum[wn * QB + 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3)] = lsum[r];
  }
  __syncthreads();
  float* rec = nparts > 1 ? part + ((static_cast<size_t>(blockIdx.z) * gridDim.y + h) * gridDim.x +
                                    blockIdx.x) * QB * attn_prefill_part_floats(HD)
                          : nullptr;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 32 * wm + 8 * (r >> 2) + 4 * hl + (r & 3);
    const int p = p0 + row;
    if (p < n) {
      const float l = ((rsum[row] + rsum[QB + row]) + rsum[2 * QB + row]) + rsum[3 * QB + row];
      if (rec) {
        float* rp = rec + static_cast<size_t>(row) * attn_prefill_part_floats(HD);
        rp[32 * wn + li] = o[r];
        if (wn == 0 && li == 0) {
          rp[HD] = m[r];
          rp[HD + 1] = l;
        }
      } else {
        out[static_cast<size_t>(p) * ldo + h * HD + 32 * wn + li] = o[r] / l;
      }
    }
  }
}

// Combines the nparts partial records of every row (grid: row blocks x
// heads, 256 threads): o = sum_i w_i o_i / sum_i w_i l_i with
// w_i = exp(m_i - max_j m_j), parts in order.  The part holding key 0 has a
// finite maximum for every row, so the overall one is finite; a part whose
// keys are all masked for a row (or that has no keys) has m_i = -inf and
// w_i = 0.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill_merge8(const float* __restrict__ part,
                                                             float* __restrict__ out, int ldo,
                                                             int n, int nparts) {
  const int p0 = blockIdx.x * kPrefillQB, h = blockIdx.y;
  constexpr size_t RF = attn_prefill_part_floats(HD);
  const size_t stride = static_cast<size_t>(gridDim.y) * gridDim.x * kPrefillQB * RF;
  const float* r0 = part + (static_cast<size_t>(h) * gridDim.x + blockIdx.x) * kPrefillQB * RF;
  constexpr int C4 = HD / 4;  // float4 columns per row
  for (int i = threadIdx.x; i < kPrefillQB * C4; i += 256) {
    const int row = i / C4, c = 4 * (i % C4);
    const int p = p0 + row;
    if (p >= n) continue;
    const float* a = r0 + row * RF;
    float mm = -INFINITY;
    for (int k = 0; k < nparts; ++k) mm = fmaxf(mm, a[k * stride + HD]);
    float l = 0.f;
    pf4 o = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nparts; ++k) {
      const float* b = a + k * stride;
      const float mk = b[HD];
      const float w = mk == -INFINITY ? 0.f : expf(mk - mm);
      l += w * b[HD + 1];
      o += w * *reinterpret_cast<const pf4*>(b + c);
    }
    *reinterpret_cast<pf4*>(out + static_cast<size_t>(p) * ldo + h * HD + c) = o * (1.f / l);
  }
}

__host__ __device__ constexpr size_t attn_prefill_mfma8_lds_bytes(int hd) {
  return (static_cast<size_t>(kPrefillKB8) * (hd + 4) +
          static_cast<size_t>(kPrefillQB) * (kPrefillKB8 + 4) + 8 * kPrefillQB) *
         sizeof(float);
}

__host__ __device__ constexpr size_t attn_prefill_mfma_lds_bytes(int hd) {
  return (2 * static_cast<size_t>(kPrefillKB) * (hd + 4) +
          static_cast<size_t>(kPrefillQB) * (kPrefillKB + 4) + 4 * kPrefillQB) *
         sizeof(float);
}

}  // namespace kl
