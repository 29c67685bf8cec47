// Wave-level GEMV cores for batch-1 decode (HBM-bound: every weight byte is
// read exactly once per token).
//
// One wave64 owns R rows (given as row pointers, so the rows may come from
// different matrices, e.g. W1 and W3 side by side).  Each lane walks the
// columns in 16-byte chunks (fp32: 4 values, int8: 16 values) with a stride of
// 64 chunks, so one wave-wide load instruction reads 1 KiB of a row
// contiguously; U chunks per row are issued back to back before any use, which
// keeps R*U independent 16-byte loads in flight per lane.  The activation
// vector x is read from LDS (the fused kernels stage it there) or from global
// memory (it is tiny and cache resident).  The caller reduces the per-lane
// partial sums across the wave.
#pragma once
#include "device.hpp"

namespace kl {

// fp32 rows.  Requires cols % 4 == 0 and 16-byte aligned rows and x.
template <int R, int U>
__device__ __forceinline__ void gemv_ptrs_f32(const float* const (&rows)[R], int cols,
                                              const float* __restrict__ x, float (&out)[R]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int c4n = cols >> 2;
  const f4* xv = reinterpret_cast<const f4*>(x);
  const f4* wr[R];
  f4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    wr[r] = reinterpret_cast<const f4*>(rows[r]);
    acc[r] = f4{0.f, 0.f, 0.f, 0.f};
  }
  int c = lane;
  for (; c + kWave * (U - 1) < c4n; c += kWave * U) {
    f4 ws[R][U];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) ws[r][u] = load_stream(wr[r] + c + kWave * u);
    f4 xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) xs[u] = xv[c + kWave * u];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) acc[r] += ws[r][u] * xs[u];
  }
  for (; c < c4n; c += kWave) {
    const f4 xs = xv[c];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] += load_stream(wr[r] + c) * xs;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = hsum(acc[r]);
}

// int8 rows with one fp32 scale per `gs` consecutive elements of the flattened
// matrix (the reference layout; since cols % gs == 0 a group never straddles
// rows, so srows[r] points at row r's first scale).  Requires gs % 16 == 0
// with gs / 16 a power of two (chunk_shift = log2(gs / 16)) and 16-byte
// aligned rows and x.  Each lane accumulates sum(x * q) over its 16-value
// chunk, then multiplies by the chunk's group scale.
template <int R, int U>
__device__ __forceinline__ void gemv_ptrs_q8(const int8_t* const (&rows)[R],
                                             const float* const (&srows)[R], int cols,
                                             int chunk_shift, const float* __restrict__ x,
                                             float (&out)[R]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int c16n = cols >> 4;
  const f4* xv = reinterpret_cast<const f4*>(x);
  const i4* wr[R];
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    wr[r] = reinterpret_cast<const i4*>(rows[r]);
    acc[r] = 0.f;
  }
  auto chunk_dot = [](const i4 w, const f4* xc) {
    float q[16];
    unpack_i8x4(w.x, q);
    unpack_i8x4(w.y, q + 4);
    unpack_i8x4(w.z, q + 8);
    unpack_i8x4(w.w, q + 12);
    f4 p = xc[0] * f4{q[0], q[1], q[2], q[3]};
    p += xc[1] * f4{q[4], q[5], q[6], q[7]};
    p += xc[2] * f4{q[8], q[9], q[10], q[11]};
    p += xc[3] * f4{q[12], q[13], q[14], q[15]};
    return hsum(p);
  };
  int c = lane;
  for (; c + kWave * (U - 1) < c16n; c += kWave * U) {
    i4 ws[R][U];
    float ss[R][U];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ws[r][u] = load_stream(wr[r] + c + kWave * u);
        ss[r][u] = srows[r][(c + kWave * u) >> chunk_shift];
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      f4 xc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) xc[k] = xv[4 * (c + kWave * u) + k];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += chunk_dot(ws[r][u], xc) * ss[r][u];
    }
  }
  for (; c < c16n; c += kWave) {
    f4 xc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) xc[k] = xv[4 * c + k];
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] += chunk_dot(load_stream(wr[r] + c), xc) * srows[r][c >> chunk_shift];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = acc[r];
}

// Weight view used by the fused kernels: fp32 (s == nullptr) or int8 + scales.
struct WView {
  const void* w;
  const float* s;
};

// R consecutive rows row0 .. row0+R-1 of one matrix; rows past nrows repeat
// the last valid row (their results are discarded by the caller).
template <bool Q8, int R, int U>
__device__ __forceinline__ void gemv_rows(WView m, int cols, int chunk_shift, int row0, int nrows,
                                          const float* x, float (&out)[R]) {
  if constexpr (Q8) {
    const int8_t* rp[R];
    const float* sp[R];
    const int gpr = (cols >> 4) >> chunk_shift;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t rr = static_cast<size_t>(row0 + (r < nrows ? r : nrows - 1));
      rp[r] = static_cast<const int8_t*>(m.w) + rr * cols;
      sp[r] = m.s + rr * gpr;
    }
    gemv_ptrs_q8<R, U>(rp, sp, cols, chunk_shift, x, out);
  } else {
    const float* rp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t rr = static_cast<size_t>(row0 + (r < nrows ? r : nrows - 1));
      rp[r] = static_cast<const float*>(m.w) + rr * cols;
    }
    gemv_ptrs_f32<R, U>(rp, cols, x, out);
  }
}

// The same RH rows of two matrices A and B streamed together (2*RH rows in
// flight): outa[r] = A[row0 + r] . x, outb[r] = B[row0 + r] . x.
template <bool Q8, int RH, int U>
__device__ __forceinline__ void gemv_rows_pair(WView A, WView B, int cols, int chunk_shift,
                                               int row0, int nrows, const float* x,
                                               float (&outa)[RH], float (&outb)[RH]) {
  float o[2 * RH];
  if constexpr (Q8) {
    const int8_t* rp[2 * RH];
    const float* sp[2 * RH];
    const int gpr = (cols >> 4) >> chunk_shift;
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const size_t rr = static_cast<size_t>(row0 + (r < nrows ? r : nrows - 1));
      rp[r] = static_cast<const int8_t*>(A.w) + rr * cols;
      sp[r] = A.s + rr * gpr;
      rp[RH + r] = static_cast<const int8_t*>(B.w) + rr * cols;
      sp[RH + r] = B.s + rr * gpr;
    }
    gemv_ptrs_q8<2 * RH, U>(rp, sp, cols, chunk_shift, x, o);
  } else {
    const float* rp[2 * RH];
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const size_t rr = static_cast<size_t>(row0 + (r < nrows ? r : nrows - 1));
      rp[r] = static_cast<const float*>(A.w) + rr * cols;
      rp[RH + r] = static_cast<const float*>(B.w) + rr * cols;
    }
    gemv_ptrs_f32<2 * RH, U>(rp, cols, x, o);
  }
#pragma unroll
  for (int r = 0; r < RH; ++r) {
    outa[r] = o[r];
    outb[r] = o[RH + r];
  }
}

}  // namespace kl
