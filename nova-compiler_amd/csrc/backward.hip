// Backward ops of the path for gfx950: nova.sce_backward, nova.layer_norm_
// backward and the column sums of nova.linear_backward's bias gradient.  All
// are HBM-bound streams (no MFMA): rows are read with coalesced 16-byte
// loads, row reductions run inside one wave64 with cross-lane shuffles, and
// column reductions over rows are deterministic -- each workgroup sums a
// fixed set of rows in a fixed order into per-workgroup partials, which a
// second pass adds up in workgroup order -- so two runs give the same bits.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "nova_hip_internal.h"
#include "wave.h"

namespace nova_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// nova.sce_backward (NovaSceBackwardLowering, NovaToLinalgGeneric.cpp:
// 1012-1137): grad = (softmax + scatter(-1 at the label)) * invN, with invN
// the f32 rounding of 1.0 / rows (one multiply per element, :1121-1128).
// A label outside [0, C) makes that row's gradient NaN.
// Grid: x = chunks of kU * 256 float4s of a row, y = rows.
// ---------------------------------------------------------------------------
struct SceBwdArgs {
  const float *softmax;
  const int32_t *labels;
  float *grad;
  int64_t ss, sg;  // row strides (elements)
  int rows, C;
  float invN;
};

// float4 chunks per thread.  One per thread over a grid of one workgroup per
// 4 KB, the fastest form of a plain copy on MI355X, runs config 5's backward
// at 164.4 against 172.8 us with four per thread (8192 x 50304: 513 against
// 552 us; the same bits).
constexpr int kU = 1;

template <bool VEC>
__global__ __launch_bounds__(256) void sce_backward_kernel(SceBwdArgs a) {
  const int row = blockIdx.y;
  const int t = a.labels[row];
  const bool bad = t < 0 || t >= a.C;
  const float nan = __builtin_nanf("");
  const float *sr = a.softmax + (int64_t)row * a.ss;
  float *gr = a.grad + (int64_t)row * a.sg;
  if constexpr (VEC) {
    const int n4 = a.C >> 2;
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(sr);
    f32x4 *g4 = reinterpret_cast<f32x4 *>(gr);
    const int base = blockIdx.x * (256 * kU) + threadIdx.x;
    f32x4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = base + 256 * u;
      v[u] = c < n4 ? __builtin_nontemporal_load(s4 + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int c = base + 256 * u;
      if (c < n4) {
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = (4 * c + e == t) ? v[u][e] + -1.0f : v[u][e];
          o[e] = bad ? nan : d * a.invN;
        }
        __builtin_nontemporal_store(o, g4 + c);
      }
    }
    // C % 4 tail: the first chunk's first threads.
    if (blockIdx.x == 0 && threadIdx.x < (a.C & 3)) {
      const int c = (n4 << 2) + threadIdx.x;
      const float d = (c == t) ? sr[c] + -1.0f : sr[c];
      gr[c] = bad ? nan : d * a.invN;
    }
  } else {
    const int base = blockIdx.x * (256 * kU * 4) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < 4 * kU; ++u) {
      const int c = base + 256 * u;
      if (c < a.C) {
        const float d = (c == t) ? sr[c] + -1.0f : sr[c];
        gr[c] = bad ? nan : d * a.invN;
      }
    }
  }
}

// Contiguous rows (row strides == C, C % 4 == 0, aligned): the matrix is one
// flat stream of float4 chunks, chunk c in row c / (C/4), so no block is
// left partly idle at a row's end.
__global__ __launch_bounds__(256) void sce_backward_flat_kernel(SceBwdArgs a, int total4) {
  const int n4 = a.C >> 2;
  const f32x4 *s4 = reinterpret_cast<const f32x4 *>(a.softmax);
  f32x4 *g4 = reinterpret_cast<f32x4 *>(a.grad);
  const int base = blockIdx.x * (256 * kU) + threadIdx.x;
  f32x4 v[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int c = base + 256 * u;
    v[u] = c < total4 ? __builtin_nontemporal_load(s4 + c) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int c = base + 256 * u;
    if (c < total4) {
      const int row = c / n4;
      const int t = a.labels[row];
      const bool bad = t < 0 || t >= a.C;
      const int e0 = 4 * (c - row * n4);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = (e0 + e == t) ? v[u][e] + -1.0f : v[u][e];
        o[e] = bad ? __builtin_nanf("") : d * a.invN;
      }
      __builtin_nontemporal_store(o, g4 + c);
    }
  }
}

// ---------------------------------------------------------------------------
// nova.layer_norm_backward (NovaLayerNormBackwardPattern,
// NovaToLinalgGeneric.cpp:2128-2371).  Per row, with the forward's saved
// S (mean_sum) and rstd and invD = 1.0f / D:
//   gg = gy * gamma; xh = (x - S*invD) * rstd
//   s1 = sum gg, s2 = sum gg * xh                        (row reductions)
//   dx = ((gg - s1*invD) - xh * (s2*invD)) * rstd        (reference op order)
//   dgamma[d] = sum_r gy * xh, dbeta[d] = sum_r gy       (column reductions)
// Each workgroup takes a fixed set of rows and writes its column sums as
// one partial [2][D] to [grid][2][D]; reduce_partials adds the partials in
// workgroup order.
// ---------------------------------------------------------------------------
struct LnBwdArgs {
  const float *gy;
  const float *x;
  const float *gamma;
  const float *mean_sum;
  const float *rstd;
  float *dx;       // may be null
  float *partial;  // [grid][2][D]
  int64_t sgy, sx, sdx;
  int rows, D;
  float invD;
};

// Each row is split over a group of four waves, wave q holding float4
// chunks [q*64*NQ, (q+1)*64*NQ) of gy and x (NQ per lane) and register
// accumulators for the same columns, so the column sums need no LDS
// traffic and no turn-taking; the row reductions s1, s2 combine the four
// waves' partials through LDS in wave order (one barrier per row).  A
// 512-thread workgroup runs two such groups on the two rows of each of its
// row pairs (pairs b, b + grid, b + 2 * grid, ... for workgroup b); at the
// end group 1's column sums are added to group 0's through LDS, and the
// workgroup writes one partial [2][D].
template <int NQ, bool FULL>
__global__ __launch_bounds__(512) void layer_norm_bwd_rows_kernel(LnBwdArgs a) {
#pragma clang fp contract(off)
  __shared__ float red[2][8][2];
  __shared__ f32x4 xfer[2][256 * NQ];
  const int nv4 = a.D >> 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave >> 2, q = wave & 3;
  auto in_row = [&](int c) __attribute__((always_inline)) { return FULL || c < nv4; };
  const f32x4 *gam4 = reinterpret_cast<const f32x4 *>(a.gamma);
  f32x4 gm[NQ], acc_g[NQ], acc_b[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    acc_g[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc_b[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Row pairs interleaved over the grid (workgroup b takes pairs b,
  // b + grid, ...): the rows in work at any time form one window that
  // sweeps the matrix in order.
  const int step = 2 * gridDim.x;
  const int row0 = 2 * blockIdx.x;
  const int row_end = a.rows;
  // Loads of row r: gy, x, the saved mean sum and rstd.  A row past the
  // matrix's end reads its last row and a chunk past the row's end
  // reads its last chunk (valid memory; the values are masked or discarded
  // where they are used), so that no load sits under a branch: a load issued
  // on one path only makes every later wait assume nothing else is in flight
  // and drain the loads of the rows ahead.  The caller guarantees
  // row0 < row_end and D >= 4.
  auto load_row = [&](int row, f32x4 (&g)[NQ], f32x4 (&xv)[NQ], float &msum, float &rs)
                      __attribute__((always_inline)) {
    const int rc = min(row, row_end - 1);
    const f32x4 *gr = reinterpret_cast<const f32x4 *>(a.gy + (int64_t)rc * a.sgy);
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(a.x + (int64_t)rc * a.sx);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int c = q * 64 * NQ + lane + 64 * i;
      const int cc = FULL ? c : min(c, nv4 - 1);
      g[i] = __builtin_nontemporal_load(gr + cc);
      xv[i] = __builtin_nontemporal_load(xr + cc);
    }
    msum = a.mean_sum[rc];
    rs = a.rstd[rc];
  };
  // With NQ <= 4 the row pairs two steps ahead are loaded while the
  // current one is reduced and written (three register slots; the loop is
  // unrolled by three so that slots are compile-time registers).  The
  // barrier waits for LDS only, not for these loads.
  constexpr bool kAhead = NQ <= 4;
  constexpr int kSlots = kAhead ? 3 : 1;
  f32x4 G[kSlots][NQ], X[kSlots][NQ];
  float Mn[kSlots], Rs[kSlots];
  int it = 0;
  // One row pair: row rb + grp, its data in slot S.
  auto pair = [&](auto slot, int rb) __attribute__((always_inline)) {
    constexpr int S = decltype(slot)::value;
    const int row = rb + grp;
    const bool live = row < row_end;
    if constexpr (kAhead) load_row(rb + 2 * step + grp, G[(S + 2) % 3], X[(S + 2) % 3],
                                   Mn[(S + 2) % 3], Rs[(S + 2) % 3]);
    else load_row(row, G[0], X[0], Mn[0], Rs[0]);
    // Chunks past the row's end count as zeros.
    f32x4 g[NQ], xv[NQ], gmv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const bool in = in_row(q * 64 * NQ + lane + 64 * i);
      g[i] = in ? G[S][i] : f32x4{0.f, 0.f, 0.f, 0.f};
      xv[i] = in ? X[S][i] : f32x4{0.f, 0.f, 0.f, 0.f};
      gmv[i] = in ? gm[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float mean = Mn[S] * a.invD, rs = Rs[S];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < NQ; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gg = g[i][e] * gmv[i][e];
        const float xh = (xv[i][e] - mean) * rs;
        s1 = s1 + gg;
        s2 = s2 + gg * xh;
      }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const int pb = it & 1;
    if (lane == 0) {
      red[pb][wave][0] = s1;
      red[pb][wave][1] = s2;
    }
    __syncthreads();
    s1 = 0.0f;
    s2 = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      s1 = s1 + red[pb][grp * 4 + w][0];
      s2 = s2 + red[pb][grp * 4 + w][1];
    }
    const float ms1 = s1 * a.invD, ms2 = s2 * a.invD;
    if (live) {
      f32x4 *dr = reinterpret_cast<f32x4 *>(a.dx + (int64_t)row * a.sdx);
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int c = q * 64 * NQ + lane + 64 * i;
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gg = g[i][e] * gmv[i][e];
          const float xh = (xv[i][e] - mean) * rs;
          const float t1 = gg - ms1;
          const float t2 = xh * ms2;
          o[e] = (t1 - t2) * rs;
          acc_g[i][e] = acc_g[i][e] + g[i][e] * xh;
          acc_b[i][e] = acc_b[i][e] + g[i][e];
        }
        if (a.dx && in_row(c)) __builtin_nontemporal_store(o, dr + c);
      }
    }
    ++it;
  };
  // One guard around the first loads and the loop: a path that enters the
  // loop without the first loads would leave gamma's loads as the only ones
  // in flight on it, and the loop's waits would be set for that path.
  if (row0 < row_end) {
    // Gamma first, ahead of the rows' loads, so that its wait is covered by
    // the first row's.
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int c = q * 64 * NQ + lane + 64 * i;
      gm[i] = gam4[FULL ? c : min(c, nv4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kAhead) {
      // In order, as the loop issues them: the loop's waits count on it.
      load_row(row0 + grp, G[0], X[0], Mn[0], Rs[0]);
      __builtin_amdgcn_sched_barrier(0);
      load_row(row0 + step + grp, G[1], X[1], Mn[1], Rs[1]);
      __builtin_amdgcn_sched_barrier(0);
      // Uniform trip count; pairs past row_end do nothing but the barrier.
      for (int rb = row0; rb < row_end; rb += 3 * step) {
        pair(std::integral_constant<int, 0>{}, rb);
        pair(std::integral_constant<int, 1>{}, rb + step);
        pair(std::integral_constant<int, 2>{}, rb + 2 * step);
      }
    } else {
      for (int rb = row0; rb < row_end; rb += step) pair(std::integral_constant<int, 0>{}, rb);
    }
  }
  // Group 1's column sums join group 0's (group 0 held the earlier row of
  // every pair), then group 0 writes the workgroup's partial.
  if (grp == 1) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      xfer[0][q * 64 * NQ + lane + 64 * i] = acc_g[i];
      xfer[1][q * 64 * NQ + lane + 64 * i] = acc_b[i];
    }
  }
  __syncthreads();
  if (grp == 0) {
    f32x4 *pg = reinterpret_cast<f32x4 *>(a.partial + (int64_t)blockIdx.x * 2 * a.D);
    f32x4 *pb = reinterpret_cast<f32x4 *>(a.partial + (int64_t)blockIdx.x * 2 * a.D + a.D);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int c = q * 64 * NQ + lane + 64 * i;
      if (in_row(c)) {
        pg[c] = acc_g[i] + xfer[0][c];
        pb[c] = acc_b[i] + xfer[1][c];
      }
    }
  }
}

// Any D (no alignment): one wave per row, elements strided by the lane; the
// column sums go through the same ordered LDS accumulation (D <= 8192 so
// the accumulators fit), two passes over the row (the second from cache).
constexpr int kAnyMaxD = 8192;

__global__ __launch_bounds__(256) void layer_norm_bwd_any_kernel(LnBwdArgs a) {
#pragma clang fp contract(off)
  __shared__ float acc_g[kAnyMaxD], acc_b[kAnyMaxD];
  for (int d = threadIdx.x; d < a.D; d += 256) {
    acc_g[d] = 0.0f;
    acc_b[d] = 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per_wg = (a.rows + gridDim.x - 1) / gridDim.x;
  const int row0 = min(a.rows, (int)blockIdx.x * per_wg);
  const int row_end = min(a.rows, row0 + per_wg);
  for (int rb = row0; rb < row_end; rb += 4) {
    const int row = rb + wave;
    const bool live = row < row_end;
    const float *gr = a.gy + (int64_t)(live ? row : row0) * a.sgy;
    const float *xr = a.x + (int64_t)(live ? row : row0) * a.sx;
    const float mean = live ? a.mean_sum[row] * a.invD : 0.0f;
    const float rs = live ? a.rstd[row] : 0.0f;
    float s1 = 0.0f, s2 = 0.0f;
    if (live) {
      for (int d = lane; d < a.D; d += 64) {
        const float gg = gr[d] * a.gamma[d];
        const float xh = (xr[d] - mean) * rs;
        s1 = s1 + gg;
        s2 = s2 + gg * xh;
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float ms1 = s1 * a.invD, ms2 = s2 * a.invD;
    if (live && a.dx) {
      float *dr = a.dx + (int64_t)row * a.sdx;
      for (int d = lane; d < a.D; d += 64) {
        const float gg = gr[d] * a.gamma[d];
        const float xh = (xr[d] - mean) * rs;
        const float t1 = gg - ms1;
        const float t2 = xh * ms2;
        dr[d] = (t1 - t2) * rs;
      }
    }
#pragma unroll 1
    for (int turn = 0; turn < 4; ++turn) {
      __syncthreads();
      if (turn == wave && live) {
        for (int d = lane; d < a.D; d += 64) {
          const float xh = (xr[d] - mean) * rs;
          acc_g[d] = acc_g[d] + gr[d] * xh;
          acc_b[d] = acc_b[d] + gr[d];
        }
      }
    }
  }
  __syncthreads();
  float *pg = a.partial + (int64_t)blockIdx.x * 2 * a.D;
  for (int d = threadIdx.x; d < a.D; d += 256) {
    pg[d] = acc_g[d];
    pg[a.D + d] = acc_b[d];
  }
}

// ---------------------------------------------------------------------------
// Column sums of a [rows, cols] matrix (f32 / bf16 / f16), stage 1: workgroup
// (x, y) sums rows [y*chunk, (y+1)*chunk) of columns [256x, 256x+256) in row
// order, one column per thread, into part[y][cols] (f32).
// ---------------------------------------------------------------------------
constexpr int kColBatch = 16;  // rows in flight per thread in the column sums

template <int DT>
__global__ __launch_bounds__(256) void col_sum_partial_kernel(const void *in, int64_t ld, int rows,
                                                              int cols, int chunk, float *part) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  const int r0 = blockIdx.y * chunk;
  const int r1 = min(rows, r0 + chunk);
  auto load = [&](int r) __attribute__((always_inline)) -> float {
    const int64_t i = (int64_t)r * ld + c;
    if constexpr (DT == NOVA_HIP_DT_F32) {
      return static_cast<const float *>(in)[i];
    } else {
      const uint16_t h = static_cast<const uint16_t *>(in)[i];
      if constexpr (DT == NOVA_HIP_DT_BF16) return __uint_as_float((uint32_t)h << 16);
      else return (float)__builtin_bit_cast(_Float16, h);
    }
  };
  // Rows go out kColBatch at a time and are added in row order (a load-add
  // loop waited out one memory latency per row).
  float acc = 0.0f;
  int r = r0;
  for (; r + kColBatch <= r1; r += kColBatch) {
    float v[kColBatch];
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) v[u] = load(r + u);
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) acc = v[u] + acc;
  }
  for (; r < r1; ++r) acc = load(r) + acc;
  part[(int64_t)blockIdx.y * cols + c] = acc;
}

// The same with 16-byte loads: each thread sums V = 16 / element-size
// adjacent columns (needs 16-byte aligned rows and cols % V == 0).
template <int DT>
__global__ __launch_bounds__(256) void col_sum_partial_vec_kernel(const void *in, int64_t ld,
                                                                  int rows, int cols, int chunk,
                                                                  float *part) {
  constexpr int V = DT == NOVA_HIP_DT_F32 ? 4 : 8;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * V;
  if (c0 >= cols) return;
  const int r0 = blockIdx.y * chunk;
  const int r1 = min(rows, r0 + chunk);
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  const char *base = static_cast<const char *>(in);
  constexpr int esz = DT == NOVA_HIP_DT_F32 ? 4 : 2;
  auto add_row = [&](const u32x4 &w) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float x;
      if constexpr (DT == NOVA_HIP_DT_F32) {
        x = __uint_as_float(w[v]);
      } else {
        const uint16_t h = (uint16_t)(w[v >> 1] >> (16 * (v & 1)));
        if constexpr (DT == NOVA_HIP_DT_BF16) x = __uint_as_float((uint32_t)h << 16);
        else x = (float)__builtin_bit_cast(_Float16, h);
      }
      acc[v] = x + acc[v];
    }
  };
  auto row_ptr = [&](int r) __attribute__((always_inline)) {
    return reinterpret_cast<const u32x4 *>(base + ((int64_t)r * ld + c0) * esz);
  };
  // Rows go out kColBatch at a time and are added in row order (a load-add
  // loop waited out one memory latency per row).
  int r = r0;
  for (; r + kColBatch <= r1; r += kColBatch) {
    u32x4 w[kColBatch];
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) w[u] = *row_ptr(r + u);
    // All loads before the first add (for f16 the scheduler otherwise
    // moved half of them down, each with its own wait).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kColBatch; ++u) add_row(w[u]);
  }
  for (; r < r1; ++r) add_row(*row_ptr(r));
  float *out = part + (int64_t)blockIdx.y * cols + c0;
#pragma unroll
  for (int v = 0; v < V; ++v) out[v] = acc[v];
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// out[c] = v in dtype odt (nothing when out is null).
__device__ __forceinline__ void store_col(void *out, int c, float v, int odt) {
  if (!out) return;
  if (odt == NOVA_HIP_DT_F32) static_cast<float *>(out)[c] = v;
  else if (odt == NOVA_HIP_DT_BF16) static_cast<uint16_t *>(out)[c] = f32_to_bf16(v);
  else static_cast<uint16_t *>(out)[c] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Stage 2 (shared by the LayerNorm and bias gradients): out_k[c] =
// sum_p part[p][k][c] over the np partials in order, for the nk outputs k
// of each partial (stride np_stride elements between partials), stored in
// dtype odt.  Thread per (k, c).
__global__ __launch_bounds__(256) void col_reduce_kernel(const float *part, int np, int nk,
                                                         int cols, int64_t p_stride, void *out0,
                                                         void *out1, int odt) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= nk * cols) return;
  const int k = idx / cols, c = idx - k * cols;
  const float *p = part + (int64_t)k * cols + c;
  float acc = 0.0f;
  int i = 0;
  // Loads issued eight ahead; the sum stays sequential in partial order.
  for (; i + 8 <= np; i += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(i + u) * p_stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = acc + v[u];
  }
  for (; i < np; ++i) acc = acc + p[(int64_t)i * p_stride];
  store_col(k == 0 ? out0 : out1, c, acc, odt);
}

// Two-level reduction of np partials when np is large: groups of kGroup
// partials are summed in order into np / kGroup second-level partials.
constexpr int kGroup = 32;

__global__ __launch_bounds__(256) void col_group_kernel(const float *part, int np, int width,
                                                        float *out) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= width) return;
  const int g = blockIdx.y;
  const int p0 = g * kGroup, p1 = min(np, p0 + kGroup);
  float acc = 0.0f;
  if (p1 - p0 == kGroup) {
    // A full group: all loads in flight at once, then the sum in partial
    // order (a load-add loop waited out one memory latency per partial).
    float v[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) v[u] = part[(int64_t)(p0 + u) * width + idx];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) acc = acc + v[u];
  } else {
    for (int p = p0; p < p1; ++p) acc = acc + part[(int64_t)p * width + idx];
  }
  out[(int64_t)g * width + idx] = acc;
}

// One launch for np <= kTreeGroups * kGroup partials: a workgroup's 256
// threads are kTreeCols columns x kTreeGroups groups; thread (g, c) sums
// partials [g * kGroup, (g + 1) * kGroup) of column c in order, all loads in
// flight at once, and the group sums are added in group order through LDS.
// That is the order of col_group_kernel followed by col_reduce_kernel, so
// the sums are the same bits, with one launch and one memory latency less.
constexpr int kTreeGroups = 8;
constexpr int kTreeCols = 256 / kTreeGroups;

__global__ __launch_bounds__(256) void col_tree_kernel(const float *part, int np, int nk,
                                                       int cols, void *out0, void *out1,
                                                       int odt) {
  __shared__ float red[kTreeGroups][kTreeCols];
  const int width = nk * cols;
  const int cl = threadIdx.x % kTreeCols, g = threadIdx.x / kTreeCols;
  const int idx = blockIdx.x * kTreeCols + cl;
  const int p0 = g * kGroup, p1 = min(np, p0 + kGroup);
  float acc = 0.0f;
  if (idx < width) {
    if (p1 - p0 == kGroup) {
      float v[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) v[u] = part[(int64_t)(p0 + u) * width + idx];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) acc = acc + v[u];
    } else {
      for (int p = p0; p < p1; ++p) acc = acc + part[(int64_t)p * width + idx];
    }
  }
  red[g][cl] = acc;
  __syncthreads();
  if (g != 0 || idx >= width) return;
  const int ng = (np + kGroup - 1) / kGroup;
  float t = 0.0f;
  for (int j = 0; j < ng; ++j) t = t + red[j][cl];
  const int k = idx / cols, c = idx - k * cols;
  store_col(k == 0 ? out0 : out1, c, t, odt);
}

// Final column reduction of np partials, each `width` = nk * cols floats
// ([np][nk][cols]); uses ws2 (np / kGroup + 1) * width floats when np is
// large.
int32_t reduce_partials(const float *part, int np, int nk, int cols, void *out0, void *out1,
                        int odt, float *ws2, hipStream_t s) {
  const int width = nk * cols;
  const unsigned blocks = (unsigned)((width + 255) / 256);
  if (np > 2 * kGroup && np <= kTreeGroups * kGroup) {
    hipLaunchKernelGGL(col_tree_kernel, dim3((unsigned)((width + kTreeCols - 1) / kTreeCols)),
                       dim3(256), 0, s, part, np, nk, cols, out0, out1, odt);
    return check_hip(hipGetLastError(), "column reduce launch");
  }
  if (np > 2 * kGroup) {
    const int ng = (np + kGroup - 1) / kGroup;
    hipLaunchKernelGGL(col_group_kernel, dim3(blocks, (unsigned)ng), dim3(256), 0, s, part, np,
                       width, ws2);
    int32_t rc = check_hip(hipGetLastError(), "column group launch");
    if (rc) return rc;
    part = ws2;
    np = ng;
  }
  hipLaunchKernelGGL(col_reduce_kernel, dim3(blocks), dim3(256), 0, s, part, np, nk, cols,
                     (int64_t)width, out0, out1, odt);
  return check_hip(hipGetLastError(), "column reduce launch");
}

}  // namespace

int32_t launch_sce_backward(const SceBackwardProblem &p, hipStream_t s) {
  if (p.rows == 0) return NOVA_HIP_SUCCESS;
  if (p.rows > 0x7fffffff || p.C > 0x7fffffff - 4096)
    return fail(NOVA_HIP_ERANGE, "sce_backward: size exceeds 2^31-1");
  SceBwdArgs a;
  a.softmax = p.softmax;
  a.labels = p.labels;
  a.grad = p.grad;
  a.ss = p.ss;
  a.sg = p.sg;
  a.rows = (int)p.rows;
  a.C = (int)p.C;
  a.invN = (float)(1.0 / (double)p.rows);
  const bool vec = aligned16(p.softmax) && aligned16(p.grad) && p.ss % 4 == 0 && p.sg % 4 == 0;
  const int64_t total4 = p.rows * (p.C / 4);
  if (vec && p.C % 4 == 0 && p.ss == p.C && p.sg == p.C && total4 < 0x7fffffff - 256 * kU) {
    const unsigned g = (unsigned)((total4 + 256 * kU - 1) / (256 * kU));
    hipLaunchKernelGGL(sce_backward_flat_kernel, dim3(g), dim3(256), 0, s, a, (int)total4);
    return check_hip(hipGetLastError(), "sce_backward launch");
  }
  // Rows beyond 65535 go in several launches (grid y limit).
  for (int64_t r0 = 0; r0 < p.rows; r0 += 65535) {
    const int64_t nr = p.rows - r0 < 65535 ? p.rows - r0 : 65535;
    SceBwdArgs b = a;
    b.softmax = p.softmax + r0 * p.ss;
    b.grad = p.grad + r0 * p.sg;
    b.labels = p.labels + r0;
    if (vec) {
      const unsigned gx = (unsigned)((p.C / 4 + 256 * kU - 1) / (256 * kU));
      hipLaunchKernelGGL(sce_backward_kernel<true>, dim3(gx > 0 ? gx : 1, (unsigned)nr),
                         dim3(256), 0, s, b);
    } else {
      const unsigned gx = (unsigned)((p.C + 256 * kU * 4 - 1) / (256 * kU * 4));
      hipLaunchKernelGGL(sce_backward_kernel<false>, dim3(gx, (unsigned)nr), dim3(256), 0, s, b);
    }
    int32_t rc = check_hip(hipGetLastError(), "sce_backward launch");
    if (rc) return rc;
  }
  return NOVA_HIP_SUCCESS;
}

int32_t launch_layer_norm_backward(const LayerNormBackwardProblem &p, hipStream_t s) {
  // The column accumulators of a workgroup live in LDS: rows up to 8192.
  // Row indices run up to three grid strides past the last row (the row
  // kernel's lookahead): rows stay below 2^31 - 2^20.
  if (p.rows > 0x7fffffff - (1 << 20))
    return fail(NOVA_HIP_ERANGE, "layer_norm_backward: %lld rows exceed 2^31 - 2^20",
                (long long)p.rows);
  if (p.D > kAnyMaxD)
    return fail(NOVA_HIP_ERANGE, "layer_norm_backward: D = %lld exceeds %d", (long long)p.D,
                kAnyMaxD);
  const bool vec = p.D % 4 == 0 && p.sgy % 4 == 0 && p.sx % 4 == 0 && (!p.dx || p.sdx % 4 == 0) &&
                   aligned16(p.gy) && aligned16(p.x) && aligned16(p.gamma) &&
                   (!p.dx || aligned16(p.dx));
  // Persistent grid, as many workgroups as fit the CUs at once, each taking
  // a fixed set of rows (every grid-th row pair in the vector kernel, one
  // contiguous block in the general one): the vector kernel's 512-thread
  // workgroups (two
  // row groups of four waves) at 2 per CU for D <= 1024 and 1 per CU above
  // (their registers, with the next row pair in flight, leave room for one),
  // the general kernel's 256-thread ones at 3 per CU.
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const bool use_vec = vec && p.D >= 4 && p.D <= 8192;
  const int64_t want = use_vec ? (p.rows + 1) / 2 : (p.rows + 3) / 4;
  const int per_cu = !use_vec ? 3 : (p.D <= 1024 ? 2 : 1);
  const int64_t cap = (int64_t)per_cu * cus;
  const int grid = (int)(want < cap ? (want > 0 ? want : 1) : cap);
  const int ng = (grid + kGroup - 1) / kGroup;
  const size_t part_floats = (size_t)grid * 2 * p.D;
  const size_t ws_floats = part_floats + (size_t)(ng + 1) * 2 * p.D;
  WorkspaceLease lease(s, ws_floats * 4);  // held until the column sums are enqueued
  float *ws = static_cast<float *>(lease.get());
  if (!ws) return NOVA_HIP_ENOMEM;
  LnBwdArgs a;
  a.gy = p.gy;
  a.x = p.x;
  a.gamma = p.gamma;
  a.mean_sum = p.mean_sum;
  a.rstd = p.rstd;
  a.dx = p.dx;
  a.partial = ws;
  a.sgy = p.sgy;
  a.sx = p.sx;
  a.sdx = p.sdx;
  a.rows = (int)p.rows;
  a.D = (int)p.D;
  a.invD = 1.0f / (float)p.D;
  if (use_vec && p.D == 1024)
    hipLaunchKernelGGL((layer_norm_bwd_rows_kernel<1, true>), dim3(grid), dim3(512), 0, s, a);
  else if (use_vec && p.D <= 1024)
    hipLaunchKernelGGL((layer_norm_bwd_rows_kernel<1, false>), dim3(grid), dim3(512), 0, s, a);
  else if (use_vec && p.D == 4096)
    hipLaunchKernelGGL((layer_norm_bwd_rows_kernel<4, true>), dim3(grid), dim3(512), 0, s, a);
  else if (use_vec && p.D <= 4096)
    hipLaunchKernelGGL((layer_norm_bwd_rows_kernel<4, false>), dim3(grid), dim3(512), 0, s, a);
  else if (use_vec)
    hipLaunchKernelGGL((layer_norm_bwd_rows_kernel<8, false>), dim3(grid), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(layer_norm_bwd_any_kernel, dim3(grid), dim3(256), 0, s, a);
  int32_t rc = check_hip(hipGetLastError(), "layer_norm_backward launch");
  if (rc) return rc;
  if (!p.dgamma && !p.dbeta) return NOVA_HIP_SUCCESS;
  return reduce_partials(ws, grid, 2, (int)p.D, p.dgamma, p.dbeta, NOVA_HIP_DT_F32,
                         ws + part_floats, s);
}

bool col_sum_in_range(int64_t rows, int64_t cols) {
  // A row chunk's end (chunk start + chunk, chunks up to 2^16 rows) and a
  // thread's first column (up to 8 per thread past the last) stay in int.
  return rows <= 0x7fffffff - (1 << 20) && cols <= 0x7fffffff - (1 << 20);
}

int32_t launch_col_sum(const ColSumProblem &p, hipStream_t s) {
  if (p.cols == 0) return NOVA_HIP_SUCCESS;
  if (!col_sum_in_range(p.rows, p.cols))
    return fail(NOVA_HIP_ERANGE, "column sum: [%lld, %lld] exceeds 2^31 - 2^20",
                (long long)p.rows, (long long)p.cols);
  // Row chunks of 64 (at most 65535 of them).
  int64_t chunk = 64;
  while ((p.rows + chunk - 1) / chunk > 65535) chunk *= 2;
  const int nch = (int)((p.rows + chunk - 1) / chunk > 0 ? (p.rows + chunk - 1) / chunk : 1);
  const int ng = (nch + kGroup - 1) / kGroup;
  const size_t part_floats = (size_t)nch * p.cols;
  WorkspaceLease lease(s, (part_floats + (size_t)(ng + 1) * p.cols) * 4);
  float *ws = static_cast<float *>(lease.get());
  if (!ws) return NOVA_HIP_ENOMEM;
  const int esz = p.in_dt == NOVA_HIP_DT_F32 ? 4 : 2;
  const int V = 16 / esz;
  if (aligned16(p.in) && (p.ld * esz) % 16 == 0 && p.cols % V == 0) {
    const dim3 gv((unsigned)((p.cols / V + 255) / 256), (unsigned)nch);
    if (p.in_dt == NOVA_HIP_DT_F32)
      hipLaunchKernelGGL(col_sum_partial_vec_kernel<NOVA_HIP_DT_F32>, gv, dim3(256), 0, s, p.in,
                         p.ld, (int)p.rows, (int)p.cols, (int)chunk, ws);
    else if (p.in_dt == NOVA_HIP_DT_BF16)
      hipLaunchKernelGGL(col_sum_partial_vec_kernel<NOVA_HIP_DT_BF16>, gv, dim3(256), 0, s, p.in,
                         p.ld, (int)p.rows, (int)p.cols, (int)chunk, ws);
    else
      hipLaunchKernelGGL(col_sum_partial_vec_kernel<NOVA_HIP_DT_F16>, gv, dim3(256), 0, s, p.in,
                         p.ld, (int)p.rows, (int)p.cols, (int)chunk, ws);
    int32_t rc = check_hip(hipGetLastError(), "column sum launch");
    if (rc) return rc;
    return reduce_partials(ws, nch, 1, (int)p.cols, p.out, nullptr, p.out_dt, ws + part_floats, s);
  }
  const dim3 g1((unsigned)((p.cols + 255) / 256), (unsigned)nch);
  if (p.in_dt == NOVA_HIP_DT_F32)
    hipLaunchKernelGGL(col_sum_partial_kernel<NOVA_HIP_DT_F32>, g1, dim3(256), 0, s, p.in, p.ld,
                       (int)p.rows, (int)p.cols, (int)chunk, ws);
  else if (p.in_dt == NOVA_HIP_DT_BF16)
    hipLaunchKernelGGL(col_sum_partial_kernel<NOVA_HIP_DT_BF16>, g1, dim3(256), 0, s, p.in, p.ld,
                       (int)p.rows, (int)p.cols, (int)chunk, ws);
  else
    hipLaunchKernelGGL(col_sum_partial_kernel<NOVA_HIP_DT_F16>, g1, dim3(256), 0, s, p.in, p.ld,
                       (int)p.rows, (int)p.cols, (int)chunk, ws);
  int32_t rc = check_hip(hipGetLastError(), "column sum launch");
  if (rc) return rc;
  return reduce_partials(ws, nch, 1, (int)p.cols, p.out, nullptr, p.out_dt, ws + part_floats, s);
}

}  // namespace nova_hip
