// Causal attention of a batch of prompt positions for the batched prefill:
// the semantics of kernels/cpu/mha_kernel.cpp:5-61 (per head h, kv head
// h / kv_mul: softmax_t((q_h . K_t) / sqrt(hd)) . V_t over t <= position) for
// query positions pos0 .. pos0 + n - 1 at once, reading K and V rows 0 ..
// pos0 + n - 1 of one layer's caches ([seq_len][kv_dim]).
//
// VALU kernel (head sizes 32 and 256): one workgroup (256 threads) owns 64
// query rows of one head and walks the key positions in blocks of KB (64; 32
// for head size 256) through LDS with an online softmax: thread (rg, cg) =
// (tid / 16, tid % 16) scores rows 4 rg .. 4 rg + 3 against keys
// KB/16 cg .. of the block, the 16 threads of a row group combine the row
// maxima and sums with lane shuffles, and the same thread accumulates output
// columns cg * HD / 16 .. of its 4 rows.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>

namespace kl {

typedef float pf4 __attribute__((ext_vector_type(4)));

constexpr int kPrefillQB = 64;  // query rows per workgroup
constexpr int kPrefillKB = 64;  // key positions per block

// Keys per block of the VALU kernel: 64, or 32 for head size 256 so that the
// Q, K and V tiles fit the 160 KB of LDS (142 KB).
__host__ __device__ constexpr int attn_prefill_kb(int hd) { return hd > 128 ? 32 : kPrefillKB; }

__host__ __device__ constexpr size_t attn_prefill_lds_bytes(int hd) {
  return (static_cast<size_t>(kPrefillQB + 2 * attn_prefill_kb(hd)) * (hd + 4) +
          static_cast<size_t>(kPrefillQB) * (attn_prefill_kb(hd) + 4)) * sizeof(float);
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ q, int ldq,
                                                      const float* __restrict__ kc,
                                                      const float* __restrict__ vc, int kv_dim,
                                                      int kv_mul, float* __restrict__ out, int ldo,
                                                      int pos0, int n, float scale) {
  constexpr int QB = kPrefillQB, KB = attn_prefill_kb(HD), LD = HD + 4, LP = KB + 4, DPT = HD / 16;
  constexpr int KPT = KB / 16;  // keys per thread and block
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
    float s[4][KPT];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < KPT; ++b) s[a][b] = 0.f;
    for (int d = 0; d < HD; d += 4) {
      pf4 qv[4], kv[KPT];
#pragma unroll
      for (int a = 0; a < 4; ++a) qv[a] = *reinterpret_cast<const pf4*>(Qs + (4 * rg + a) * LD + d);
#pragma unroll
      for (int b = 0; b < KPT; ++b) kv[b] = *reinterpret_cast<const pf4*>(Ks + (KPT * cg + b) * LD + d);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < KPT; ++b)
          s[a][b] += qv[a].x * kv[b].x + qv[a].y * kv[b].y + qv[a].z * kv[b].z + qv[a].w * kv[b].w;
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int qpos = pos0 + p0 + 4 * rg + a;
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < KPT; ++b) {
        const int kpos = j0 + KPT * cg + b;
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
      for (int b = 0; b < KPT; ++b) {
        const float pv = s[a][b] == -INFINITY ? 0.f : expf(s[a][b] - mn);
        Ps[(4 * rg + a) * LP + KPT * cg + b] = pv;
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

// Head sizes 64 and 128 on the matrix cores: FlashAttention-2 style on
// v_mfma_f32_16x16x4f32 with no exchange between waves inside a key block
// (head size 128 runs k_attn_prefill_x6 below unless KL_PREFILL_ATTN=f32).
// A workgroup of eight waves takes 64 query rows of one head and walks key
// blocks of 64: wave w computes for query rows 16 (w % 4) .. + 15 and the
// keys of half w / 4 of every block, two waves per SIMD; the two halves'
// running (max, sum, output) merge once at the end.  Each wave computes
// S^T = K Q^T and O^T += V^T P^T, so that in the 16 x 16 accumulator layout
// (register r of lane l holds row 4 (l / 16) + r, column l % 16) every score
// and every output value a lane holds belongs to query l % 16: the row
// maximum and sum need only the lane's 8 scores of a block and two lane
// exchanges (xor 16, 32), and the rescaling of O and the P operand of O^T stay
// in registers (P^T's accumulator register r of a 16-key sub-block is the B
// operand of step r, key 4 (l / 16) + r of the sub-block).  Lane group
// g = l / 16 takes d columns HD/4 g .. of the scores' k dimension (its Q row
// slice in registers), in two halves with their own accumulators so that
// consecutive MFMAs are independent.  Row i of O^T block b is
// d = 64 (b / 4) + 4 i + b % 4: the A operand of step r for blocks
// 4 hb .. 4 hb + 3 is then one 16-byte read of V row (key) 4 (l / 16) + r at
// d = 64 hb + 4 (l % 16), and a lane ends holding 16 consecutive output
// columns 64 hb + 16 (l / 16) .. of its query.
//
// K and V are both staged row-major [key][d] by direct-to-LDS loads (no
// register staging), unpadded, 16-byte chunk c of row r at slot
// c ^ fa_swz<HD>(r).  A 16-byte LDS read is served half a wave (32 lanes) at a
// time over 512 B of banks; the swizzle puts the 32 lanes of a K read (16
// consecutive rows, chunks c and c + HD/16) and of a V read (rows R and R + 4,
// 16 consecutive chunks each) on distinct slots (head size 64: the K reads;
// its V rows R and R + 4 share a 512-byte window whatever the swizzle).  K of
// the next block is requested as soon as
// every wave has its scores, V of a block once every wave is done with the
// previous one; two barriers per key block.  Scores are kept in base 2
// (scale log2 e) for the native exponential.
//
// Work decomposition.  A unit is one (head h, 64-row block i, 64-key block
// kb) triple; the units of row block i of head h form segment h nqb + i (key
// blocks 0 .. (last position of the row block) / 64).  Without a workspace,
// workgroup s takes segment s whole.  With one (stream-K), G workgroups take
// equal contiguous ranges [w W / G, (w + 1) W / G) of the W units in segment
// order, so every CU walks the same number of key blocks however unequal the
// causal segments are.  A segment cut by a range boundary leaves one partial
// record per piece (unnormalised output row, natural-log max, sum; slot 0 for
// the piece that starts the workgroup's range, slot 1 for the one that ends
// it), combined in key order by k_attn_prefill_merge; a piece whose keys all
// come after a row's position leaves that row max -inf, sum 0.
constexpr int kFaKB = 64;          // keys per block
constexpr int kFaMaxWorkers = 256; // stream-K workgroups (one per CU of an MI355X)
static_assert(kFaKB == kPrefillQB, "row blocks and key blocks share the 64 grid");

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Chunk swizzle of the K/V tiles (see above).  Head size 128 (512-byte rows,
// 32 chunks): bits 0, 1, 2, 4 = bits 0, 1, 3, 2 of r.  Head size 64 (256-byte
// rows, 16 chunks): bits 0, 1, 2, 3 = bits 1, 2, 0, 3 of r.  Both depend on
// r mod 16 only and are a bijection of the row's chunks.
template <int HD>
__host__ __device__ constexpr int fa_swz(int r) {
  return HD == 128 ? (r & 3) | ((r >> 1) & 4) | ((r & 4) << 2)
                   : ((r >> 1) & 3) | ((r & 1) << 2) | (r & 8);
}

// One partial record per query row: HD output floats, then max and sum,
// padded to a multiple of 4 floats so that every record (and every float4
// column group the merge reads) starts 16-byte aligned.
__host__ __device__ constexpr size_t attn_prefill_part_floats(int hd) { return hd + 4; }

__host__ __device__ constexpr size_t attn_prefill_fa_lds_bytes(int hd) {
  return 2 * static_cast<size_t>(kFaKB) * hd * sizeof(float);
}

// Stream-K workspace: two record slots of 64 rows per workgroup.
__host__ __device__ constexpr size_t attn_prefill_fa_ws_bytes(int hd) {
  return 2 * static_cast<size_t>(kFaMaxWorkers) * kPrefillQB * attn_prefill_part_floats(hd) *
         sizeof(float);
}

// Unit geometry of a launch over query positions pos0 .. pos0 + n - 1.
struct FaGeom {
  int nqb;        // 64-row blocks
  int a;          // key blocks of row block 0; row block i < nqb - 1 has a + i
  int nk_last;    // key blocks of the last row block
  long long wh;   // units per head
};
__host__ __device__ inline long long fa_seg_start(const FaGeom& g, long long i) {
  return i * g.a + i * (i - 1) / 2;
}
__host__ __device__ inline int fa_seg_len(const FaGeom& g, int i) {
  return i < g.nqb - 1 ? g.a + i : g.nk_last;
}
__host__ __device__ inline FaGeom fa_geom(int pos0, int n) {
  FaGeom g;
  g.nqb = (n + kPrefillQB - 1) / kPrefillQB;
  g.a = (pos0 + kPrefillQB - 1) / kFaKB + 1;
  g.nk_last = (pos0 + n - 1) / kFaKB + 1;
  g.wh = fa_seg_start(g, g.nqb - 1) + g.nk_last;
  return g;
}
// Row block of the segment holding unit r (0 <= r < wh) of a head: the
// largest i < nqb with fa_seg_start(i) <= r (a root estimate, then exact).
__device__ inline int fa_locate(const FaGeom& g, long long r) {
  const double b = g.a - 0.5;
  long long i = static_cast<long long>(sqrt(b * b + 2.0 * static_cast<double>(r)) - b);
  i = i < 0 ? 0 : (i > g.nqb - 1 ? g.nqb - 1 : i);
  while (i > 0 && fa_seg_start(g, i) > r) --i;
  while (i < g.nqb - 1 && fa_seg_start(g, i + 1) <= r) ++i;
  return static_cast<int>(i);
}
// Workgroup whose range holds unit u (W units over G workgroups).
__host__ __device__ inline long long fa_worker(long long u, long long W, long long G) {
  return ((u + 1) * G - 1) / W;
}

template <int HD>
__global__ __launch_bounds__(512) void k_attn_prefill_fa(const float* __restrict__ q, int ldq,
                                                         const float* __restrict__ kc,
                                                         const float* __restrict__ vc, int kv_dim,
                                                         int kv_mul, float* __restrict__ out,
                                                         int ldo, int pos0, int n, float scale,
                                                         int heads, float* __restrict__ part) {
  static_assert(HD == 64 || HD == 128, "head size");
  constexpr int QB = kPrefillQB, KB = kFaKB, NT = 512;
  constexpr int DG = HD / 4;       // d columns per lane group (scores)
  constexpr int DC = DG / 4;       // their float4 chunks
  constexpr int NB = HD / 16;      // 16-row blocks of O^T
  constexpr int NH = HD / 64;      // 64-column groups of a V row
  constexpr int C4 = HD / 4;       // 16-byte chunks per K / V row
  constexpr int LI = KB * C4 / NT; // 1 KB direct-to-LDS loads per wave and operand
  constexpr int LDO = HD + 4;      // merge record row: o[HD], m, l
  constexpr size_t RF = attn_prefill_part_floats(HD);
  static_assert(QB == 64 && KB == 64 && DC % 2 == 0 && KB * C4 % NT == 0, "tile");
  static_assert(static_cast<size_t>(QB) * LDO <= 2 * static_cast<size_t>(KB) * HD,
                "merge records fit the K/V buffers");
  extern __shared__ __align__(1024) float sm[];
  float* Ks = sm;            // [KB][HD], chunk c of row r at slot c ^ fa_swz<HD>(r)
  float* Vs = sm + KB * HD;  // same layout
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave & 3, kh = wave >> 2;  // query group, key half
  const int lg = lane >> 4, l16 = lane & 15;
  const FaGeom geo = fa_geom(pos0, n);
  // This workgroup's unit range [u0, u1) and the segment (h, i) holding u0.
  long long u0, u1;
  int h, i;
  if (part) {
    const long long W = geo.wh * heads, G = gridDim.x;
    u0 = blockIdx.x * W / G;
    u1 = (blockIdx.x + 1) * W / G;
    h = static_cast<int>(u0 / geo.wh);
    i = fa_locate(geo, u0 - h * geo.wh);
  } else {
    h = static_cast<int>(blockIdx.x) / geo.nqb;
    i = static_cast<int>(blockIdx.x) % geo.nqb;
    u0 = h * geo.wh + fa_seg_start(geo, i);
    u1 = u0 + fa_seg_len(geo, i);
  }
  long long seg = h * geo.wh + fa_seg_start(geo, i);  // first unit of segment (h, i)
  // Direct-to-LDS load u of this wave fills tile chunks 64 (LI wave + u) + lane:
  // row r = that / C4, slot s = that % C4, which holds chunk s ^ fa_swz(r).
  int drow[LI], dofs[LI];
#pragma unroll
  for (int u = 0; u < LI; ++u) {
    const int P = 64 * (LI * wave + u) + lane;
    const int r = P / C4, s = P % C4;
    drow[u] = r;
    dofs[u] = 4 * (s ^ fa_swz<HD>(r));
  }
  const int kswz = fa_swz<HD>(l16);  // the swizzle of every K row this lane reads
  const float scale2 = scale * 1.44269504088896340736f;
  for (long long u = u0; u < u1;) {
    const int len = fa_seg_len(geo, i);
    const long long e = u1 < seg + len ? u1 : seg + len;
    const int kbA = static_cast<int>(u - seg), kbB = static_cast<int>(e - seg);
    const int p0 = QB * i;
    const int rows = n - p0 < QB ? n - p0 : QB;
    const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
    const float* kg = kc + (h / kv_mul) * HD;
    const float* vg = vc + (h / kv_mul) * HD;
    // Rows past `last` read row `last` (their scores are masked, p = 0).
    auto request = [&](const float* src, float* dst, int j0) {
#pragma unroll
      for (int t = 0; t < LI; ++t) {
        const int row = j0 + drow[t] <= last ? j0 + drow[t] : last;
        __builtin_amdgcn_global_load_lds(
            (global_void_t*)(src + static_cast<size_t>(row) * kv_dim + dofs[t]),
            (lds_void_t*)(dst + 256 * (LI * wave + t)), 16, 0, 0);
      }
    };
    __syncthreads();  // the previous piece's merge records are read
    request(kg, Ks, kbA * KB);
    const int qrow = p0 + 16 * qg + l16;  // this lane's query (rows past n: not stored)
    const int qpos = pos0 + (qrow < n ? qrow : n - 1);
    pf4 qr[DC];
    {
      const float* qp = q + static_cast<size_t>(qrow < n ? qrow : 0) * ldq + h * HD + DG * lg;
#pragma unroll
      for (int c = 0; c < DC; ++c)
        qr[c] = qrow < n ? *reinterpret_cast<const pf4*>(qp + 4 * c) : pf4{0.f, 0.f, 0.f, 0.f};
    }
    float m = -INFINITY, l = 0.f;  // running maximum (base 2) and sum of this key half
    pf4 oacc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) oacc[b] = pf4{0.f, 0.f, 0.f, 0.f};
    for (int kb = kbA; kb < kbB; ++kb) {
      const int j0 = kb * KB;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();  // K of this block landed; V of the previous one consumed
      request(vg, Vs, j0);
      // S^T[key][query] for keys 16 (2 kh + k) + 4 lg + r of the block, the d
      // range in two halves with their own accumulators.
      pf4 sacc[2][2];
#pragma unroll
      for (int k = 0; k < 2; ++k) sacc[k][0] = sacc[k][1] = pf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c2 = 0; c2 < DC / 2; ++c2) {
        pf4 kf[2][2];
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int dh = 0; dh < 2; ++dh) {
            const int r = 16 * (2 * kh + k) + l16;
            const int c = DC * lg + c2 + dh * DC / 2;
            kf[k][dh] = *reinterpret_cast<const pf4*>(Ks + r * HD + 4 * (c ^ kswz));
          }
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
#pragma unroll
          for (int dh = 0; dh < 2; ++dh)
#pragma unroll
            for (int k = 0; k < 2; ++k)
              sacc[k][dh] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  kf[k][dh][e4], qr[c2 + dh * DC / 2][e4], sacc[k][dh], 0, 0, 0);
      }
      pf4 sc[2];
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = j0 + 16 * (2 * kh + k) + 4 * lg + r;
          const float v = sacc[k][0][r] + sacc[k][1][r];
          sc[k][r] = key <= qpos ? v * scale2 : -INFINITY;
          mx = fmaxf(mx, sc[k][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m, mx);
      // A key half with no key at or before the row yet keeps max -inf, sum 0.
      const float alpha = m == -INFINITY ? 0.f : exp2f(m - mn);
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = sc[k][r];
          const float pv = v == -INFINITY ? 0.f : exp2f(v - mn);
          sc[k][r] = pv;
          sum += pv;
        }
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      l = l * alpha + sum;
      m = mn;
#pragma unroll
      for (int b = 0; b < NB; ++b) oacc[b] *= alpha;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();  // V landed; every wave's K reads of this block done
      if (kb + 1 < kbB) request(kg, Ks, j0 + KB);
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int r = 16 * (2 * kh + k) + 4 * lg + r4;
          pf4 vf[NH];
#pragma unroll
          for (int hb = 0; hb < NH; ++hb)
            vf[hb] = *reinterpret_cast<const pf4*>(Vs + r * HD + 4 * ((16 * hb + l16) ^ fa_swz<HD>(r)));
#pragma unroll
          for (int b = 0; b < NB; ++b)
            oacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[b / 4][b % 4], sc[k][r4], oacc[b], 0,
                                                           0, 0);
        }
    }
    // Output columns 64 hb + 16 lg + 4 r .. + 3 of this lane's query.
    auto cols = [&](int hb, int r) {
      return pf4{oacc[4 * hb][r], oacc[4 * hb + 1][r], oacc[4 * hb + 2][r], oacc[4 * hb + 3][r]};
    };
    // Merge the key halves: half 1 leaves (o, m, l) in LDS, half 0 combines.
    __syncthreads();  // the last block's K and V are consumed
    float* rec = sm + (16 * qg + l16) * LDO;
    if (kh == 1) {
#pragma unroll
      for (int hb = 0; hb < NH; ++hb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<pf4*>(rec + 64 * hb + 16 * lg + 4 * r) = cols(hb, r);
      if (lg == 0) {
        rec[HD] = m;
        rec[HD + 1] = l;
      }
    }
    __syncthreads();
    if (kh == 0 && qrow < n) {
      const float m1 = rec[HD], l1 = rec[HD + 1];
      const float mm = fmaxf(m, m1);
      const float w0 = m == -INFINITY ? 0.f : exp2f(m - mm);
      const float w1 = m1 == -INFINITY ? 0.f : exp2f(m1 - mm);
      l = l * w0 + l1 * w1;
      const bool whole = kbA == 0 && kbB == len;
      float* dst;
      if (whole) {
        dst = out + static_cast<size_t>(qrow) * ldo + h * HD;
      } else {
        dst = part + ((2 * static_cast<size_t>(blockIdx.x) + (u == u0 ? 0 : 1)) * QB + (qrow - p0)) * RF;
        if (lg == 0) {
          dst[HD] = mm * 0.69314718055994530942f;  // natural units for the merge
          dst[HD + 1] = l;
        }
      }
#pragma unroll
      for (int hb = 0; hb < NH; ++hb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 64 * hb + 16 * lg + 4 * r;
          pf4 o = cols(hb, r) * w0 + *reinterpret_cast<const pf4*>(rec + d) * w1;
          if (whole) o = o / l;
          *reinterpret_cast<pf4*>(dst + d) = o;
        }
    }
    u = e;
    seg += len;
    if (++i == geo.nqb) {
      i = 0;
      ++h;
    }
  }
}

// Combines the pieces of every segment that stream-K cut: thread t of a
// 256-thread workgroup takes float4 column t % (HD / 4) of one row (grid:
// row groups x heads); o = sum_k w_k o_k / sum_k w_k l_k with
// w_k = exp(m_k - max_j m_j) over the pieces in key order.  The piece holding
// key 0 has a finite maximum for every row, so the overall one is finite; a
// piece whose keys are all masked for a row has m_k = -inf and w_k = 0.
// Segments left whole were written by the attention kernel.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill_merge(const float* __restrict__ part,
                                                            float* __restrict__ out, int ldo,
                                                            int pos0, int n, int heads,
                                                            int workers) {
  constexpr int TPR = HD / 4, RPB = 256 / TPR, GPB = kPrefillQB / RPB;  // threads per row, rows per workgroup
  constexpr size_t RF = attn_prefill_part_floats(HD);
  const int i = blockIdx.x / GPB, h = blockIdx.y;
  const int row = RPB * (blockIdx.x % GPB) + threadIdx.x / TPR, c = 4 * (threadIdx.x % TPR);
  const FaGeom geo = fa_geom(pos0, n);
  const long long W = geo.wh * heads, G = workers;
  const long long s0 = h * geo.wh + fa_seg_start(geo, i), s1 = s0 + fa_seg_len(geo, i);
  const long long wa = fa_worker(s0, W, G), wb = fa_worker(s1 - 1, W, G);
  const int p = kPrefillQB * i + row;
  if (wa == wb || p >= n) return;
  // The first piece is slot 1 of its workgroup unless the segment starts that
  // workgroup's range; every later piece starts its workgroup's range.
  const int slot_a = s0 > wa * W / G ? 1 : 0;
  const float* r0 = part + ((2 * static_cast<size_t>(wa) + slot_a) * kPrefillQB + row) * RF;
  const float* r1 = part + (2 * static_cast<size_t>(wa + 1) * kPrefillQB + row) * RF;
  const size_t step = 2 * kPrefillQB * RF;  // one workgroup's records
  auto rec = [&](long long w) { return w == wa ? r0 : r1 + (w - wa - 1) * step; };
  float mm = -INFINITY;
  for (long long w = wa; w <= wb; ++w) mm = fmaxf(mm, rec(w)[HD]);
  float l = 0.f;
  pf4 o = {0.f, 0.f, 0.f, 0.f};
  for (long long w = wa; w <= wb; ++w) {
    const float* b = rec(w);
    const float mk = b[HD];
    const float wk = mk == -INFINITY ? 0.f : expf(mk - mm);
    l += wk * b[HD + 1];
    o += wk * *reinterpret_cast<const pf4*>(b + c);
  }
  *reinterpret_cast<pf4*>(out + static_cast<size_t>(p) * ldo + h * HD + c) = o * (1.f / l);
}


// Head size 128 with the products as split bf16 terms: k_attn_prefill_fa's
// decomposition (stream-K units, eight waves, query group w % 4 and key half
// w / 4, S^T = K Q^T and O^T += V^T P^T in the 16 x 16 accumulator layout, the
// key halves merged at the end, the same partial records) with each product
// on v_mfma_f32_16x16x32_bf16 as the six terms Xi Yj, i + j <= 2, of the
// operands split into three bf16 planes x = x0 + x1 + x2 (x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1), round to nearest even; the split
// of k_split3), which carry all 24 significand bits: the terms left out are
// each at most 2^-24 |x y|, so scores and outputs are as accurate as on the
// fp32 matrix cores, at 16x the rate per product.
//
// Per key block every thread loads 16 floats of K (key t / 8, d 16 (t % 8) ..)
// and 16 of V (keys 4 (t / 32) .., d 4 (t % 32) ..) into registers one block
// ahead, and after a barrier writes their planes to LDS: K key-major (rows of
// 256 B per plane, 16-byte chunk c of key r at slot c ^ ((r >> 1) & 7) 2, so
// the 32 lanes of a half wave -- 16 consecutive keys, chunks c and c + 1 --
// read 32 distinct slots of 512 B), V transposed, d-major (rows of 64 keys,
// 128 B per plane, 8-byte chunk c of row d at slot c ^ ((d >> 2) & 15)).
// A lane's S^T operand is K row 32 kh + 16 k + l % 16, d 32 j + 8 g .. + 7
// (g = l / 16) against its query's Q slice, split once per row block into
// registers.  Its scores are keys 32 kh + 16 k + 4 g + i (register i of
// sub-block k), which as P^T's B operand of one 32-key step are k-values
// 8 g + 4 k + i; the A operand (V^T) of output block b then reads, for d =
// 64 (b / 4) + 4 (l % 16) + b % 4, keys 32 kh + 4 g .. + 3 and 32 kh + 16 +
// 4 g .. + 3: two 8-byte reads of the d row.  Row 4 g + i of O^T block b is
// that d, so a lane ends holding the output columns k_attn_prefill_fa's do.
typedef __bf16 abf8 __attribute__((ext_vector_type(8)));
typedef __bf16 abf4 __attribute__((ext_vector_type(4)));
typedef float af16 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr size_t attn_prefill_x6_lds_bytes() {
  return 2 * 3 * static_cast<size_t>(kFaKB) * 128 * 2;  // K and V^T planes
}

typedef float af2 __attribute__((ext_vector_type(2)));
typedef __bf16 abf2 __attribute__((ext_vector_type(2)));

// Two values into their three planes (packed conversions, two per instruction).
__device__ __forceinline__ void x6_split2(af2 v, abf2& x0, abf2& x1, abf2& x2) {
  x0 = __builtin_convertvector(v, abf2);
  const af2 r1 = v - __builtin_convertvector(x0, af2);
  x1 = __builtin_convertvector(r1, abf2);
  x2 = __builtin_convertvector(r1 - __builtin_convertvector(x1, af2), abf2);
}

__device__ __forceinline__ void x6_split8(const float (&v)[8], abf8& x0, abf8& x1, abf8& x2) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    abf2 y0, y1, y2;
    x6_split2(af2{v[e], v[e + 1]}, y0, y1, y2);
    x0[e] = y0[0];
    x0[e + 1] = y0[1];
    x1[e] = y1[0];
    x1[e + 1] = y1[1];
    x2[e] = y2[0];
    x2[e + 1] = y2[1];
  }
}

__global__ __launch_bounds__(512) void k_attn_prefill_x6(const float* __restrict__ q, int ldq,
                                                         const float* __restrict__ kc,
                                                         const float* __restrict__ vc, int kv_dim,
                                                         int kv_mul, float* __restrict__ out,
                                                         int ldo, int pos0, int n, float scale,
                                                         int heads, float* __restrict__ part) {
  constexpr int HD = 128, QB = kPrefillQB, KB = kFaKB;
  constexpr int NB = HD / 16;      // 16-row blocks of O^T
  constexpr int NH = HD / 64;      // 64-column groups of the output
  constexpr int LDO = HD + 4;      // merge record row: o[HD], m, l
  constexpr int PK = KB * HD;      // bf16 per plane (K or V^T)
  constexpr size_t RF = attn_prefill_part_floats(HD);
  static_assert(QB == 64 && KB == 64, "tile");
  static_assert(static_cast<size_t>(QB) * LDO * sizeof(float) <= attn_prefill_x6_lds_bytes(),
                "merge records fit the plane buffers");
  extern __shared__ __align__(1024) float sm[];
  __bf16* Kp = reinterpret_cast<__bf16*>(sm);  // [3][KB][HD], swizzled 16-byte chunks
  __bf16* Vt = Kp + 3 * PK;                    // [3][HD][KB], swizzled 8-byte chunks
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave & 3, kh = wave >> 2;  // query group, key half
  const int lg = lane >> 4, l16 = lane & 15;
  const FaGeom geo = fa_geom(pos0, n);
  long long u0, u1;
  int h, i;
  if (part) {
    const long long W = geo.wh * heads, G = gridDim.x;
    u0 = blockIdx.x * W / G;
    u1 = (blockIdx.x + 1) * W / G;
    h = static_cast<int>(u0 / geo.wh);
    i = fa_locate(geo, u0 - h * geo.wh);
  } else {
    h = static_cast<int>(blockIdx.x) / geo.nqb;
    i = static_cast<int>(blockIdx.x) % geo.nqb;
    u0 = h * geo.wh + fa_seg_start(geo, i);
    u1 = u0 + fa_seg_len(geo, i);
  }
  long long seg = h * geo.wh + fa_seg_start(geo, i);
  // This thread's share of a key block: K key kr, d 16 kc16 .. + 15; V keys
  // 4 vq .. + 3, d 4 ve .. + 3.
  const int kr = tid >> 3, kc16 = tid & 7, vq = tid >> 5, ve = tid & 31;
  const float scale2 = scale * 1.44269504088896340736f;
  for (long long u = u0; u < u1;) {
    const int len = fa_seg_len(geo, i);
    const long long e = u1 < seg + len ? u1 : seg + len;
    const int kbA = static_cast<int>(u - seg), kbB = static_cast<int>(e - seg);
    const int p0 = QB * i;
    const int rows = n - p0 < QB ? n - p0 : QB;
    const int last = pos0 + p0 + rows - 1;  // last key any row of the block attends
    const float* kg = kc + (h / kv_mul) * HD;
    const float* vg = vc + (h / kv_mul) * HD;
    // Rows past `last` read row `last` (their scores are masked, p = 0).
    pf4 kreg[4], vreg[4];
    auto load = [&](int j0) {
      const int rk = j0 + kr <= last ? j0 + kr : last;
      const pf4* ks = reinterpret_cast<const pf4*>(kg + static_cast<size_t>(rk) * kv_dim + 16 * kc16);
#pragma unroll
      for (int c = 0; c < 4; ++c) kreg[c] = ks[c];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int rv = j0 + 4 * vq + c <= last ? j0 + 4 * vq + c : last;
        vreg[c] = *reinterpret_cast<const pf4*>(vg + static_cast<size_t>(rv) * kv_dim + 4 * ve);
      }
    };
    auto store = [&]() {
      const int ksw = ((kr >> 1) & 7) << 1;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float v[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = kreg[2 * hh + c / 4][c % 4];
        abf8 x[3];
        x6_split8(v, x[0], x[1], x[2]);
        const int slot = (2 * kc16 + hh) ^ ksw;
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<abf8*>(Kp + pl * PK + kr * HD + 8 * slot) = x[pl];
      }
#pragma unroll
      for (int dj = 0; dj < 4; ++dj) {
        const int d = 4 * ve + dj;
        abf2 a0, a1, a2, b0, b1, b2;
        x6_split2(af2{vreg[0][dj], vreg[1][dj]}, a0, a1, a2);
        x6_split2(af2{vreg[2][dj], vreg[3][dj]}, b0, b1, b2);
        __bf16* dst = Vt + d * KB + 4 * (vq ^ ((d >> 2) & 15));
        *reinterpret_cast<abf4*>(dst) = abf4{a0[0], a0[1], b0[0], b0[1]};
        *reinterpret_cast<abf4*>(dst + PK) = abf4{a1[0], a1[1], b1[0], b1[1]};
        *reinterpret_cast<abf4*>(dst + 2 * PK) = abf4{a2[0], a2[1], b2[0], b2[1]};
      }
    };
    load(kbA * KB);
    const int qrow = p0 + 16 * qg + l16;  // this lane's query (rows past n: not stored)
    const int qpos = pos0 + (qrow < n ? qrow : n - 1);
    abf8 qx[4][3];  // Q^T operand: d 32 j + 8 g .. + 7 of the lane's query, three planes
    {
      const float* qp = q + static_cast<size_t>(qrow < n ? qrow : 0) * ldq + h * HD + 8 * lg;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v[8];
        const pf4 a = qrow < n ? *reinterpret_cast<const pf4*>(qp + 32 * j) : pf4{0.f, 0.f, 0.f, 0.f};
        const pf4 b = qrow < n ? *reinterpret_cast<const pf4*>(qp + 32 * j + 4) : pf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v[c] = a[c];
          v[4 + c] = b[c];
        }
        x6_split8(v, qx[j][0], qx[j][1], qx[j][2]);
      }
    }
    float m = -INFINITY, l = 0.f;  // running maximum (base 2) and sum of this key half
    af16 oacc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) oacc[b] = af16{0.f, 0.f, 0.f, 0.f};
    constexpr int PX[6] = {2, 1, 0, 1, 0, 0}, PY[6] = {0, 1, 2, 0, 1, 0};  // smallest terms first
    for (int kb = kbA; kb < kbB; ++kb) {
      const int j0 = kb * KB;
      __syncthreads();  // every wave is done with the previous block's planes (and the records)
      store();
      if (kb + 1 < kbB) load(j0 + KB);
      __syncthreads();  // this block's planes are in LDS
      // S^T[key][query] for keys 32 kh + 16 k + 4 lg + r of the block.
      af16 sacc[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) sacc[k] = af16{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        abf8 kf[2][3];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int r = 32 * kh + 16 * k + l16;
          const int slot = (4 * j + lg) ^ (((r >> 1) & 7) << 1);
#pragma unroll
          for (int pl = 0; pl < 3; ++pl) kf[k][pl] = *reinterpret_cast<const abf8*>(Kp + pl * PK + r * HD + 8 * slot);
        }
#pragma unroll
        for (int t = 0; t < 6; ++t)
#pragma unroll
          for (int k = 0; k < 2; ++k)
            sacc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[k][PX[t]], qx[j][PY[t]], sacc[k], 0, 0, 0);
      }
      pf4 sc[2];
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = j0 + 16 * (2 * kh + k) + 4 * lg + r;
          const float v = sacc[k][r];
          sc[k][r] = key <= qpos ? v * scale2 : -INFINITY;
          mx = fmaxf(mx, sc[k][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m, mx);
      // A key half with no key at or before the row yet keeps max -inf, sum 0.
      const float alpha = m == -INFINITY ? 0.f : exp2f(m - mn);
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = sc[k][r];
          const float pv = v == -INFINITY ? 0.f : exp2f(v - mn);
          sc[k][r] = pv;
          sum += pv;
        }
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      l = l * alpha + sum;
      m = mn;
#pragma unroll
      for (int b = 0; b < NB; ++b) oacc[b] *= alpha;
      // P^T operand: k-value 8 lg + 4 k + r is key 32 kh + 16 k + 4 lg + r.
      abf8 pb[3];
      {
        float v[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = sc[c / 4][c % 4];
        x6_split8(v, pb[0], pb[1], pb[2]);
      }
      const int c0 = 8 * kh + lg, c1 = 8 * kh + 4 + lg;  // 4-key chunks of the V^T rows
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int d = 64 * (b / 4) + 4 * l16 + (b % 4);
        const int sw = (d >> 2) & 15;
        abf8 vf[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
          const __bf16* row = Vt + pl * PK + d * KB;
          const abf4 lo = *reinterpret_cast<const abf4*>(row + 4 * (c0 ^ sw));
          const abf4 hi = *reinterpret_cast<const abf4*>(row + 4 * (c1 ^ sw));
          vf[pl] = abf8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int t = 0; t < 6; ++t)
          oacc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[PX[t]], pb[PY[t]], oacc[b], 0, 0, 0);
      }
    }
    // Output columns 64 hb + 16 lg + 4 r .. + 3 of this lane's query.
    auto cols = [&](int hb, int r) {
      return pf4{oacc[4 * hb][r], oacc[4 * hb + 1][r], oacc[4 * hb + 2][r], oacc[4 * hb + 3][r]};
    };
    // Merge the key halves: half 1 leaves (o, m, l) in LDS, half 0 combines.
    __syncthreads();  // the last block's planes are consumed
    float* rec = sm + (16 * qg + l16) * LDO;
    if (kh == 1) {
#pragma unroll
      for (int hb = 0; hb < NH; ++hb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *reinterpret_cast<pf4*>(rec + 64 * hb + 16 * lg + 4 * r) = cols(hb, r);
      if (lg == 0) {
        rec[HD] = m;
        rec[HD + 1] = l;
      }
    }
    __syncthreads();
    if (kh == 0 && qrow < n) {
      const float m1 = rec[HD], l1 = rec[HD + 1];
      const float mm = fmaxf(m, m1);
      const float w0 = m == -INFINITY ? 0.f : exp2f(m - mm);
      const float w1 = m1 == -INFINITY ? 0.f : exp2f(m1 - mm);
      l = l * w0 + l1 * w1;
      const bool whole = kbA == 0 && kbB == len;
      float* dst;
      if (whole) {
        dst = out + static_cast<size_t>(qrow) * ldo + h * HD;
      } else {
        dst = part + ((2 * static_cast<size_t>(blockIdx.x) + (u == u0 ? 0 : 1)) * QB + (qrow - p0)) * RF;
        if (lg == 0) {
          dst[HD] = mm * 0.69314718055994530942f;  // natural units for the merge
          dst[HD + 1] = l;
        }
      }
#pragma unroll
      for (int hb = 0; hb < NH; ++hb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 64 * hb + 16 * lg + 4 * r;
          pf4 o = cols(hb, r) * w0 + *reinterpret_cast<const pf4*>(rec + d) * w1;
          if (whole) o = o / l;
          *reinterpret_cast<pf4*>(dst + d) = o;
        }
    }
    u = e;
    seg += len;
    if (++i == geo.nqb) {
      i = 0;
      ++h;
    }
  }
}

}  // namespace kl
