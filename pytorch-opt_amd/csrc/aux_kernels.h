// Memory-bound helper kernels shared by the op drivers: deterministic
// per-matrix sums of squares, LDS-tiled pack/transpose with scaling and
// zero padding, pad clearing and fills. None of these use hipMemset*, so
// every op stays safe to record into a HIP graph.
#pragma once

#include <algorithm>

#include "pto_common.h"

namespace pto {

constexpr int kRedBlocks = 1024;  // partial sums per matrix

// partial[b][blk] = sum of x^2 over rows blk, blk + kRedBlocks, ... of
// matrix b (double accumulation, fixed order, so deterministic). Rows are
// read as 16-byte runs when the pitch and base allow.
template <typename T>
__global__ void __launch_bounds__(256) sumsq_partial_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                            int64_t ld, int64_t sb, double* __restrict__ partial) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int b = blockIdx.y;
  const T* xb = x + (int64_t)b * sb;
  const bool vec = ld % VEC == 0 && (reinterpret_cast<uintptr_t>(xb) & 15) == 0;
  const int64_t nv = vec ? cols / VEC : 0;  // whole 16-byte runs per row
  double s = 0.0;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = xb + r * ld;
    for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
      const uint4 u = reinterpret_cast<const uint4*>(row)[v];
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const double d = to_f(e[k]);
        s += d * d;
      }
    }
    for (int64_t c = nv * VEC + threadIdx.x; c < cols; c += blockDim.x) {
      const double d = to_f(row[c]);
      s += d * d;
    }
  }
  __shared__ double red[256];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[(int64_t)b * gridDim.x + blockIdx.x] = red[0];
}

// Sum of matrix b's kRedBlocks partials by the whole (256-thread) block in a
// fixed order (each thread sums a strided quarter in index order, then a
// tree), so the result is deterministic. Every thread gets the sum.
__device__ __forceinline__ double block_sum_partials(const double* __restrict__ partial, int b) {
  __shared__ double red[256];
  double s = 0.0;
  for (int i = threadIdx.x; i < kRedBlocks; i += 256) s += partial[(int64_t)b * kRedBlocks + i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  return red[0];
}

template <typename T>
int launch_sumsq(const T* x, int64_t rows, int64_t cols, int64_t ld, int64_t sb, int batch, double* partial,
                 hipStream_t stream) {
  if (batch == 0) return 0;
  hipLaunchKernelGGL(sumsq_partial_kernel<T>, dim3(kRedBlocks, batch), dim3(256), 0, stream, x, rows, cols, ld, sb,
                     partial);
  PTO_LAUNCHED("sumsq_partial");
  return 0;
}

// out(r, c) = s_b * in(r, c) into a straight copy S and/or a transposed copy
// Tt, both padded: S is [rows][ld_s] with cols..ld_s zero, Tt is
// [cols + ones][ld_t] with rows..ld_t zero. If `ones` is set, Tt gets an
// extra row (index cols) equal to 1 for r < rows (an appended ones column
// of the input). scale == nullptr means s_b = 1.
template <typename TI, typename TO, typename S>
__global__ void __launch_bounds__(256) pack_kernel(const TI* __restrict__ in, int64_t rows, int64_t cols, int64_t ld_in,
                                                   int64_t s_in, const S* __restrict__ scale, TO* __restrict__ out_s,
                                                   int64_t ld_s, int64_t s_s, TO* __restrict__ out_t, int64_t ld_t,
                                                   int64_t s_t, int ones) {
  __shared__ float tile[64][65];
  const int b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const TI* ib = in + (int64_t)b * s_in;
  const S sc = scale ? scale[b] : S(1);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  // Read the (r0, c0) tile of the input, coalesced along c.
  for (int rr = ty; rr < 64; rr += 4) {
    int64_t r = r0 + rr, c = c0 + tx;
    float v = 0.f;
    if (r < rows && c < cols) v = static_cast<float>(static_cast<S>(to_f(ib[r * ld_in + c])) * sc);
    else if (ones && r < rows && c == cols) v = 1.f;
    tile[rr][tx] = v;
  }
  __syncthreads();
  if (out_s) {
    TO* ob = out_s + (int64_t)b * s_s;
    for (int rr = ty; rr < 64; rr += 4) {
      int64_t r = r0 + rr, c = c0 + tx;
      if (r < rows && c < ld_s) ob[r * ld_s + c] = static_cast<TO>(c < cols ? tile[rr][tx] : 0.f);
    }
  }
  if (out_t) {
    TO* ob = out_t + (int64_t)b * s_t;
    const int64_t trows = cols + (ones ? 1 : 0);
    for (int cc = ty; cc < 64; cc += 4) {
      int64_t c = c0 + cc, r = r0 + tx;  // output row c, output column r
      if (c < trows && r < ld_t) ob[c * ld_t + r] = static_cast<TO>(r < rows ? tile[tx][cc] : 0.f);
    }
  }
}

// Same as pack_kernel but exact for double data (the float tile would round).
template <typename TI, typename TO, typename S>
__global__ void __launch_bounds__(256) pack_kernel_f64(const TI* __restrict__ in, int64_t rows, int64_t cols,
                                                       int64_t ld_in, int64_t s_in, const S* __restrict__ scale,
                                                       TO* __restrict__ out_s, int64_t ld_s, int64_t s_s,
                                                       TO* __restrict__ out_t, int64_t ld_t, int64_t s_t, int ones) {
  __shared__ double tile[64][65];
  const int b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const TI* ib = in + (int64_t)b * s_in;
  const S sc = scale ? scale[b] : S(1);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int rr = ty; rr < 64; rr += 4) {
    int64_t r = r0 + rr, c = c0 + tx;
    double v = 0.0;
    if (r < rows && c < cols) v = static_cast<double>(static_cast<S>(to_f(ib[r * ld_in + c])) * sc);
    else if (ones && r < rows && c == cols) v = 1.0;
    tile[rr][tx] = v;
  }
  __syncthreads();
  if (out_s) {
    TO* ob = out_s + (int64_t)b * s_s;
    for (int rr = ty; rr < 64; rr += 4) {
      int64_t r = r0 + rr, c = c0 + tx;
      if (r < rows && c < ld_s) ob[r * ld_s + c] = convert<TO>(c < cols ? tile[rr][tx] : 0.0);
    }
  }
  if (out_t) {
    TO* ob = out_t + (int64_t)b * s_t;
    const int64_t trows = cols + (ones ? 1 : 0);
    for (int cc = ty; cc < 64; cc += 4) {
      int64_t c = c0 + cc, r = r0 + tx;
      if (c < trows && r < ld_t) ob[c * ld_t + r] = convert<TO>(r < rows ? tile[tx][cc] : 0.0);
    }
  }
}

// pack_kernel for 2- and 4-byte element types with 16-byte global accesses:
// each thread reads runs of VEC = 16 / sizeof elements along an input row,
// writes the straight copy from registers and the transposed copy through
// an LDS tile held transposed (tt[c][r], rows padded by VEC elements so
// that every tile row starts 16-byte aligned). Same values and padding as
// pack_kernel. Needs 16-byte aligned bases and pitches and batch strides
// that are multiples of VEC.
template <typename TI, typename TO, typename S>
__global__ void __launch_bounds__(256) pack_vec_kernel(const TI* __restrict__ in, int64_t rows, int64_t cols,
                                                       int64_t ld_in, int64_t s_in, const S* __restrict__ scale,
                                                       TO* __restrict__ out_s, int64_t ld_s, int64_t s_s,
                                                       TO* __restrict__ out_t, int64_t ld_t, int64_t s_t, int ones) {
  static_assert(sizeof(TI) == sizeof(TO) && (sizeof(TI) == 2 || sizeof(TI) == 4), "2- or 4-byte types");
  constexpr int VEC = 16 / (int)sizeof(TI);
  constexpr int CPR = 64 / VEC;  // 16-byte runs per 64-element tile row
  constexpr int P = 64 + VEC;    // LDS pitch in elements
  __shared__ __attribute__((aligned(16))) TO tt[64 * P];
  const int b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const TI* ib = in + (int64_t)b * s_in;
  const S sc = scale ? scale[b] : S(1);
  for (int q = threadIdx.x; q < 64 * CPR; q += 256) {
    const int rr = q / CPR, cc = (q % CPR) * VEC;
    const int64_t r = r0 + rr, c = c0 + cc;
    TO v[VEC];
    if (r < rows && c + VEC <= cols) {
      const uint4 u = *reinterpret_cast<const uint4*>(ib + r * ld_in + c);
      const TI* e = reinterpret_cast<const TI*>(&u);
#pragma unroll
      for (int k = 0; k < VEC; ++k) v[k] = static_cast<TO>(static_cast<float>(static_cast<S>(to_f(e[k])) * sc));
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        float x = 0.f;
        if (r < rows && c + k < cols) x = static_cast<float>(static_cast<S>(to_f(ib[r * ld_in + c + k])) * sc);
        else if (ones && r < rows && c + k == cols) x = 1.f;
        v[k] = static_cast<TO>(x);
      }
    }
    if (out_s && r < rows && c < ld_s) {  // the ones column is not part of the straight copy
      uint4 u;
      TO* w = reinterpret_cast<TO*>(&u);
#pragma unroll
      for (int k = 0; k < VEC; ++k) w[k] = c + k < cols ? v[k] : static_cast<TO>(0.f);
      *reinterpret_cast<uint4*>(out_s + (int64_t)b * s_s + r * ld_s + c) = u;
    }
    if (out_t) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) tt[(cc + k) * P + rr] = v[k];
    }
  }
  if (!out_t) return;
  __syncthreads();
  TO* ob = out_t + (int64_t)b * s_t;
  const int64_t trows = cols + (ones ? 1 : 0);
  for (int q = threadIdx.x; q < 64 * CPR; q += 256) {
    const int cc = q / CPR, rr = (q % CPR) * VEC;  // output row c0 + cc, columns r0 + rr ..
    const int64_t c = c0 + cc, r = r0 + rr;
    if (c < trows && r < ld_t)
      *reinterpret_cast<uint4*>(ob + c * ld_t + r) = *reinterpret_cast<const uint4*>(&tt[cc * P + rr]);
  }
}

// Straight copy only (no transposed output, no ones column): rows of 16-byte
// runs, out(r, c) = s_b * in(r, c) for c < cols and 0 for cols <= c < ld_out.
// Same value conversion as pack_kernel. Needs 16-byte aligned bases and
// pitches that are multiples of 16 bytes; TI and TO of the same 2- or
// 4-byte size.
template <typename TI, typename TO, typename S>
__global__ void __launch_bounds__(256) pack_rows_kernel(const TI* __restrict__ in, int64_t rows, int64_t cols,
                                                        int64_t ld_in, int64_t s_in, const S* __restrict__ scale,
                                                        TO* __restrict__ out, int64_t ld_out, int64_t s_out) {
  static_assert(sizeof(TI) == sizeof(TO) && sizeof(TI) <= 4, "same 2- or 4-byte types");
  constexpr int VEC = 16 / (int)sizeof(TI);
  const int b = blockIdx.y;
  const TI* ib = in + (int64_t)b * s_in;
  TO* ob = out + (int64_t)b * s_out;
  const S sc = scale ? scale[b] : S(1);
  const int64_t nchunk = ld_out / VEC;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const TI* irow = ib + r * ld_in;
    TO* orow = ob + r * ld_out;
    for (int64_t ch = threadIdx.x; ch < nchunk; ch += blockDim.x) {
      const int64_t c0 = ch * VEC;
      uint4 uo;
      TO* o = reinterpret_cast<TO*>(&uo);
      if (c0 + VEC <= cols) {
        const uint4 ui = reinterpret_cast<const uint4*>(irow)[ch];
        const TI* e = reinterpret_cast<const TI*>(&ui);
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = static_cast<TO>(static_cast<float>(static_cast<S>(to_f(e[k])) * sc));
      } else {
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const int64_t c = c0 + k;
          o[k] = static_cast<TO>(c < cols ? static_cast<float>(static_cast<S>(to_f(irow[c])) * sc) : 0.f);
        }
      }
      reinterpret_cast<uint4*>(orow)[ch] = uo;
    }
  }
}

// Host wrapper. The grid covers the padded extents of both outputs.
template <typename TI, typename TO, typename S>
int launch_pack(const TI* in, int64_t rows, int64_t cols, int64_t ld_in, int64_t s_in, const S* scale, TO* out_s,
                int64_t ld_s, int64_t s_s, TO* out_t, int64_t ld_t, int64_t s_t, bool ones, int batch,
                hipStream_t stream) {
  if (batch == 0) return 0;
  if constexpr (sizeof(TI) == sizeof(TO) && sizeof(TI) <= 4 && sizeof(S) == 4) {
    constexpr int VEC = 16 / (int)sizeof(TI);
    const bool rows_ok = out_t == nullptr && !ones && out_s != nullptr && ld_in % VEC == 0 && ld_s % VEC == 0 &&
                         s_in % VEC == 0 && s_s % VEC == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(out_s) & 15) == 0;
    if (rows_ok) {
      PTO_REQUIRE(batch < 65536, "pack: grid too large");
      const unsigned gx = (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, 1024));
      hipLaunchKernelGGL((pack_rows_kernel<TI, TO, S>), dim3(gx, (unsigned)batch), dim3(256), 0, stream, in, rows,
                         cols, ld_in, s_in, scale, out_s, ld_s, s_s);
      PTO_LAUNCHED("pack_rows");
      return 0;
    }
  }
  int64_t rext = rows, cext = cols + (ones ? 1 : 0);
  if (out_s) cext = std::max<int64_t>(cext, ld_s);
  if (out_t) rext = std::max<int64_t>(rext, ld_t);
  dim3 grid((unsigned)((cext + 63) / 64), (unsigned)((rext + 63) / 64), (unsigned)batch);
  PTO_REQUIRE(grid.y < 65536 && grid.z < 65536, "pack: grid too large");
  if constexpr (sizeof(TI) == sizeof(TO) && (sizeof(TI) == 2 || sizeof(TI) == 4) && sizeof(S) == 4) {
    constexpr int VEC = 16 / (int)sizeof(TI);
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vec = al(in) && ld_in % VEC == 0 && s_in % VEC == 0 &&
                     (!out_s || (al(out_s) && ld_s % VEC == 0 && s_s % VEC == 0)) &&
                     (!out_t || (al(out_t) && ld_t % VEC == 0 && s_t % VEC == 0));
    if (vec) {
      hipLaunchKernelGGL((pack_vec_kernel<TI, TO, S>), grid, dim3(256), 0, stream, in, rows, cols, ld_in, s_in,
                         scale, out_s, ld_s, s_s, out_t, ld_t, s_t, ones ? 1 : 0);
      PTO_LAUNCHED("pack_vec");
      return 0;
    }
  }
  if (sizeof(S) == 8 || sizeof(TO) == 8 || sizeof(TI) == 8)
    hipLaunchKernelGGL((pack_kernel_f64<TI, TO, S>), grid, dim3(256), 0, stream, in, rows, cols, ld_in, s_in, scale,
                       out_s, ld_s, s_s, out_t, ld_t, s_t, ones ? 1 : 0);
  else
    hipLaunchKernelGGL((pack_kernel<TI, TO, S>), grid, dim3(256), 0, stream, in, rows, cols, ld_in, s_in, scale,
                       out_s, ld_s, s_s, out_t, ld_t, s_t, ones ? 1 : 0);
  PTO_LAUNCHED("pack");
  return 0;
}

// Zero columns [c0, ld) of every row of a batched [rows][ld] buffer.
template <typename T>
__global__ void zero_cols_kernel(T* __restrict__ buf, int64_t rows, int64_t ld, int64_t c0, int64_t sb) {
  const int b = blockIdx.y;
  const int64_t w = ld - c0, total = rows * w;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e / w, c = c0 + (e - r * w);
    buf[(int64_t)b * sb + r * ld + c] = T(0);
  }
}

template <typename T>
int launch_zero_cols(T* buf, int64_t rows, int64_t ld, int64_t c0, int64_t sb, int batch, hipStream_t stream) {
  if (c0 >= ld || rows == 0 || batch == 0) return 0;
  int64_t total = rows * (ld - c0);
  unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 1024);
  hipLaunchKernelGGL(zero_cols_kernel<T>, dim3(blocks, batch), dim3(256), 0, stream, buf, rows, ld, c0, sb);
  PTO_LAUNCHED("zero_cols");
  return 0;
}

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, int64_t n, T v) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x)
    p[e] = v;
}

template <typename T>
int launch_fill(T* p, int64_t n, T v, hipStream_t stream) {
  if (n == 0) return 0;
  unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 2048);
  hipLaunchKernelGGL(fill_kernel<T>, dim3(blocks), dim3(256), 0, stream, p, n, v);
  PTO_LAUNCHED("fill");
  return 0;
}

}  // namespace pto
