// GEMV building blocks for batch-1 decode (HBM-bound: every weight byte is
// read exactly once per token).
//
// Work unit: one wave64 owns a "tile" = R rows x one column slice.  A slice
// is U 16-byte chunks per lane (fp32: 4 values/chunk, int8: 16 values/chunk),
// i.e. 64*U chunks = U KiB per row, read by U wave-wide load instructions
// that each cover 1 KiB of the row contiguously.  All R*U loads of a tile are
// issued together into registers before any of them is used, so a kernel can
// issue its first tile's weights before it stages the activation vector
// (RMSNorm prologue), and the next tile's weights before it reduces the
// current one.  A row longer than one slice is split over KS waves of the
// same workgroup (split-K) and the partial sums meet in LDS.
#pragma once
#include "device.hpp"

namespace kl {

// Weight view: fp32 (s == nullptr) or int8 + one fp32 scale per group of
// consecutive elements of the flattened matrix (the reference layout; since
// cols % group == 0 a group never straddles rows).
struct WView {
  const void* w;
  const float* s;
};

// Column geometry of one matrix for a kernel: chunks per row and how they
// split into KS slices of 64*U chunks.
struct ColGeom {
  int cols;        // values per row
  int cn;          // 16-byte chunks per row
  int ks;          // slices per row (waves per row)
  int chunk_shift; // int8: log2(chunks per scale group)
};

template <bool Q8, int U>
struct Slice;

template <int U>
struct Slice<false, U> {
  f4 w[U];
  // c0 = slice * 64 * U + lane: first chunk this lane reads.
  __device__ __forceinline__ void load(WView m, size_t row, const ColGeom& g, int c0) {
    const f4* p = reinterpret_cast<const f4*>(static_cast<const float*>(m.w) + row * g.cols);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + kWave * u;
      w[u] = c < g.cn ? load_stream(p + c) : f4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // Per-lane partial dot product with x (LDS or global), same chunk indices.
  __device__ __forceinline__ float dot(const float* x, const ColGeom& g, int c0) const {
    const f4* xv = reinterpret_cast<const f4*>(x);
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + kWave * u;
      if (c < g.cn) acc += w[u] * xv[c];
    }
    return hsum(acc);
  }
};

template <int U>
struct Slice<true, U> {
  i4 w[U];
  float s[U];
  __device__ __forceinline__ void load(WView m, size_t row, const ColGeom& g, int c0) {
    const i4* p = reinterpret_cast<const i4*>(static_cast<const int8_t*>(m.w) + row * g.cols);
    const float* sp = m.s + row * static_cast<size_t>(g.cn >> g.chunk_shift);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + kWave * u;
      const bool ok = c < g.cn;
      w[u] = ok ? load_stream(p + c) : i4{0, 0, 0, 0};
      s[u] = ok ? sp[c >> g.chunk_shift] : 0.f;
    }
  }
  __device__ __forceinline__ float dot(const float* x, const ColGeom& g, int c0) const {
    const f4* xv = reinterpret_cast<const f4*>(x);
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + kWave * u;
      if (c < g.cn) {
        const f4* xc = xv + 4 * c;
        float q[16];
        unpack_i8x4(w[u].x, q);
        unpack_i8x4(w[u].y, q + 4);
        unpack_i8x4(w[u].z, q + 8);
        unpack_i8x4(w[u].w, q + 12);
        f4 p = xc[0] * f4{q[0], q[1], q[2], q[3]};
        p += xc[1] * f4{q[4], q[5], q[6], q[7]};
        p += xc[2] * f4{q[8], q[9], q[10], q[11]};
        p += xc[3] * f4{q[12], q[13], q[14], q[15]};
        acc += hsum(p) * s[u];
      }
    }
    return acc;
  }
};

// Host-side geometry for a matrix with `cols` columns, U chunks per slice.
inline ColGeom make_geom(int cols, bool q8, int U, int group_size) {
  ColGeom g;
  g.cols = cols;
  g.cn = q8 ? cols / 16 : cols / 4;
  g.ks = (g.cn + kWave * U - 1) / (kWave * U);
  g.chunk_shift = 0;
  if (q8) {
    const int cpg = group_size / 16;
    while ((1 << g.chunk_shift) < cpg) ++g.chunk_shift;
  }
  return g;
}

// Workgroup layout for split-K tiles: KS waves per row group, G row groups;
// blockDim.x = 64 * KS * G: 256 threads for KS in {1, 2, 4}, KS waves (up to
// 8) otherwise.
inline int row_groups_for(int ks) { return ks <= 4 ? 4 / ks : 1; }
constexpr int kMaxKs = 8;

// Block-wide sum for any blockDim.x multiple of 64 (<= 1024); `red` is LDS
// scratch of >= 16 floats.  Every thread receives the total.  Contains
// barriers: call uniformly.
__device__ __forceinline__ float block_sum_any(float v, float* red) {
  v = wave_sum(v);
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < nw; ++w) t += red[w];
  return t;
}

// Stage the GEMV input in LDS, applying RMSNorm on the way when nw != null
// (kernels/cpu/rmsnorm_kernel.cpp:30-32: y = w * (x / sqrt(mean(x^2) + eps))).
// Ends with a barrier.  Call uniformly.
__device__ __forceinline__ void stage_input(const float* __restrict__ x,
                                            const float* __restrict__ nw, float eps, int n,
                                            float* xs, float* red) {
  if (nw) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const float v = x[i];
      ss += v * v;
    }
    ss = block_sum_any(ss, red);
    const float r = 1.f / sqrtf(ss / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = nw[i] * (r * x[i]);
  } else {
    for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = x[i];
  }
  __syncthreads();
}

// Drives the tiles of one GEMV-shaped kernel.  `units` row units of R rows;
// KS = g.ks waves per unit (split-K), G = blockDim.x / (64 KS) units per
// workgroup pass, grid-stride over passes.
//   rows(u, r, WView&, size_t& row): where row r of unit u lives
//   stage(): stages the input vector into xs (ends with a barrier)
//   epi(u, const float (&v)[R]): consumes the finished dot products; called
//     by every lane of one wave per unit (values are wave-uniform)
// The first pass's weights are requested before stage(), and each next
// pass's weights before the current pass is reduced.  `red` is LDS scratch of
// >= 16 * R floats.  Contains barriers: call uniformly.
template <bool Q8, int R, int U, class RowsFn, class StageFn, class EpiFn>
__device__ __forceinline__ void run_tiles(const ColGeom& g, int units, const float* xs,
                                          float* red, RowsFn rows, StageFn stage, EpiFn epi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int ks = g.ks;
  const int G = blockDim.x / (kWave * ks);
  const int slice = wave % ks;
  const int rg = wave / ks;
  const int c0 = slice * kWave * U + lane;
  const int nblk = (units + G - 1) / G;
  Slice<Q8, U> t[R];
  auto load = [&](int blk) {
    const int u = min(blk * G + rg, units - 1);  // clamped duplicates are discarded
#pragma unroll
    for (int r = 0; r < R; ++r) {
      WView m;
      size_t row;
      rows(u, r, m, row);
      t[r].load(m, row, g, c0);
    }
  };
  int b = blockIdx.x;
  if (b < nblk) load(b);
  stage();
  for (; b < nblk; b += gridDim.x) {
    float p[R];
#pragma unroll
    for (int r = 0; r < R; ++r) p[r] = t[r].dot(xs, g, c0);
    if (b + static_cast<int>(gridDim.x) < nblk) load(b + gridDim.x);
#pragma unroll
    for (int r = 0; r < R; ++r) p[r] = wave_sum(p[r]);
    const int u = b * G + rg;
    if (ks == 1) {
      if (u < units) epi(u, p);
    } else {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) red[wave * R + r] = p[r];
      }
      __syncthreads();
      if (slice == 0 && u < units) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float acc = 0.f;
          for (int k = 0; k < ks; ++k) acc += red[(rg * ks + k) * R + r];
          p[r] = acc;
        }
        epi(u, p);
      }
      __syncthreads();
    }
  }
}

}  // namespace kl
