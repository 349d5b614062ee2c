// Row reductions for gfx950: nova.layer_norm and nova.sce (softmax
// cross-entropy with mean loss).  Both are HBM-bound, so neither uses MFMA:
// rows are streamed with coalesced 16-byte loads, reduced inside one wave64
// with cross-lane shuffles, and every input byte is read once.
//
// The reference GPU pipeline gives these [parallel, reduction] generics one
// row per thread with row-strided (uncoalesced) loads and a sequential
// in-thread reduction (NovaKernelConfig.cpp:1585-1760); the CPU pipeline
// reads x twice for LayerNorm and the logits three times for SCE.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "nova_hip_internal.h"
#include "wave.h"

namespace nova_hip {
namespace {

constexpr int kWaves = 4;  // rows per 256-thread workgroup

typedef float f32x4 __attribute__((ext_vector_type(4)));


// ---------------------------------------------------------------------------
// LayerNorm.  Per row (NovaLayerNormPattern, NovaToLinalgGeneric.cpp:
// 1997-2126):  S = sum x, Q = sum x^2; mean = S*invD; var = Q*invD - mean^2;
// rstd = 1/sqrt(var + eps); y = ((x - mean) * rstd) * gamma + beta.
// The elementwise part keeps the reference's operation order (no FMA
// contraction); S and Q are summed lane-wise then across the wave.
// ---------------------------------------------------------------------------
struct LnArgs {
  const float *x;
  const float *gamma;
  const float *beta;
  float *y;
  float *mean_sum;
  float *rstd;
  int64_t sx, sy;
  int rows, D;
  float eps, invD;
};

// Row held in registers: NV f32x4 per lane covers D <= 256 * NV.  The grid
// is persistent (a few workgroups per CU): gamma and beta are staged in LDS
// once per workgroup instead of re-read from L2 for every row, and each wave
// walks rows with a grid stride.
template <int NV, bool FULL>
__global__ __launch_bounds__(256) void layer_norm_reg_kernel(LnArgs a) {
#pragma clang fp contract(off)
  __shared__ f32x4 sg[64 * NV], sb[64 * NV];
  const int nv4 = a.D >> 2;
  const f32x4 *g4 = reinterpret_cast<const f32x4 *>(a.gamma);
  const f32x4 *b4 = reinterpret_cast<const f32x4 *>(a.beta);
  for (int c = threadIdx.x; c < nv4; c += 256) {
    sg[c] = g4[c];
    sb[c] = b4[c];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  // FULL: D == 256 * NV, so every lane's NV chunks are inside the row and
  // the loads and stores need no guards (guarded, they cost ~5% here).
  auto in_row = [&](int c) __attribute__((always_inline)) { return FULL || c < nv4; };
  // Each workgroup takes a contiguous block of rows, its waves interleaved
  // inside it, so one workgroup's reads and its S / rstd writes stay close.
  const int per_wg = (a.rows + gridDim.x - 1) / gridDim.x;
  const int row_end = min(a.rows, (int)(blockIdx.x + 1) * per_wg);
  for (int row = blockIdx.x * per_wg + (threadIdx.x >> 6); row < row_end; row += kWaves) {
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(a.x + (int64_t)row * a.sx);
    f32x4 v[NV];
    float s = 0.0f, q = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      v[i] = in_row(c) ? __builtin_nontemporal_load(xr + c) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      s = s + v[i].x; s = s + v[i].y; s = s + v[i].z; s = s + v[i].w;
      q = q + v[i].x * v[i].x; q = q + v[i].y * v[i].y;
      q = q + v[i].z * v[i].z; q = q + v[i].w * v[i].w;
    }
    s = wave_sum(s);
    q = wave_sum(q);
    const float mean = s * a.invD;
    const float sq_mean = q * a.invD;
    const float mean_sq = mean * mean;
    const float var = sq_mean - mean_sq;
    const float rstd = 1.0f / sqrtf(var + a.eps);
    f32x4 *yr = reinterpret_cast<f32x4 *>(a.y + (int64_t)row * a.sy);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (in_row(c)) {
        const f32x4 g = sg[c], b = sb[c];
        f32x4 o;
        o.x = ((v[i].x - mean) * rstd) * g.x + b.x;
        o.y = ((v[i].y - mean) * rstd) * g.y + b.y;
        o.z = ((v[i].z - mean) * rstd) * g.z + b.z;
        o.w = ((v[i].w - mean) * rstd) * g.w + b.w;
        __builtin_nontemporal_store(o, yr + c);
      }
    }
    if (lane == 0) {
      if (a.mean_sum) a.mean_sum[row] = s;
      if (a.rstd) a.rstd[row] = rstd;
    }
  }
}

// Any D, any alignment: two passes over the row (the second from cache).
__global__ __launch_bounds__(256) void layer_norm_any_kernel(LnArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const float *xr = a.x + (int64_t)row * a.sx;
  float s = 0.0f, q = 0.0f;
  for (int d = lane; d < a.D; d += 64) {
    const float v = xr[d];
    s = s + v;
    q = q + v * v;
  }
  s = wave_sum(s);
  q = wave_sum(q);
  const float mean = s * a.invD;
  const float var = q * a.invD - mean * mean;
  const float rstd = 1.0f / sqrtf(var + a.eps);
  float *yr = a.y + (int64_t)row * a.sy;
  for (int d = lane; d < a.D; d += 64)
    yr[d] = ((xr[d] - mean) * rstd) * a.gamma[d] + a.beta[d];
  if (lane == 0) {
    if (a.mean_sum) a.mean_sum[row] = s;
    if (a.rstd) a.rstd[row] = rstd;
  }
}

// ---------------------------------------------------------------------------
// Softmax cross-entropy (NovaSceForwardLowering, NovaToLinalgGeneric.cpp:
// 801-1010) in one pass over the logits: per lane a running (max, sum of
// exp(x - max)) updated once per 32-value chunk, merged across the wave.
//   lse = log(max(sum, 1e-7)); loss_r = lse - (x[label] - max);
// Row losses go to a workspace; sce_mean_kernel forms the mean.
// ---------------------------------------------------------------------------
struct SceArgs {
  const float *logits;
  const int32_t *labels;
  float *loss;
  float *softmax;
  float *grad;          // fused nova.sce_backward output, or null
  float *row_loss;      // workspace [rows]
  int64_t sx, ssm, sg;
  int rows, C;
  float invN;           // f32 rounding of 1.0 / rows (NovaToLinalgGeneric.cpp:1121-1125)
};

// Gradient of the mean loss for one element from its softmax value sm:
// (sm + (-1 at the label)) * invN, the arithmetic of nova.sce_backward
// (NovaToLinalgGeneric.cpp:1102-1128) applied to the softmax this kernel
// would store.  A label outside [0, C) gives NaN.
__device__ __forceinline__ float sce_grad(float sm, bool at_label, bool bad, float invN) {
  const float d = at_label ? sm + -1.0f : sm;
  return bad ? __builtin_nanf("") : d * invN;
}

constexpr float kLog2e = 1.4426950408889634f;

// exp(x - m) as 2^((x - m) * log2e) on v_exp_f32.  The subtraction comes
// first, as in the reference (subf then math.exp), so x == m gives exactly 1.
__device__ __forceinline__ float exp_shifted(float x, float m) {
  return __builtin_amdgcn_exp2f((x - m) * kLog2e);
}

template <bool VEC>
__global__ __launch_bounds__(256) void sce_kernel(SceArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);

  if (row < a.rows) {
    const float *xr = a.logits + (int64_t)row * a.sx;
    float m = -INFINITY, s = 0.0f;
    if constexpr (VEC) {
      const f32x4 *x4 = reinterpret_cast<const f32x4 *>(xr);
      const int n4 = a.C >> 2;
      constexpr int U = 8;  // f32x4 per lane per chunk
      int base = 0;
      for (; base + 64 * U <= n4; base += 64 * U) {
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(x4 + base + lane + 64 * u);
        float cm = m;
#pragma unroll
        for (int u = 0; u < U; ++u)
          cm = fmaxf(cm, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
        float cs = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          cs += exp_shifted(v[u].x, cm);
          cs += exp_shifted(v[u].y, cm);
          cs += exp_shifted(v[u].z, cm);
          cs += exp_shifted(v[u].w, cm);
        }
        s = (m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - cm) * kLog2e)) + cs;
        m = cm;
      }
      // Tail: remaining f32x4s, then the scalar remainder.
      for (int c = base + lane; c < n4; c += 64) {
        const f32x4 v = x4[c];
        const float cm = fmaxf(m, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
        const float cs = exp_shifted(v.x, cm) + exp_shifted(v.y, cm) +
                         exp_shifted(v.z, cm) + exp_shifted(v.w, cm);
        s = (m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - cm) * kLog2e)) + cs;
        m = cm;
      }
      for (int c = (n4 << 2) + lane; c < a.C; c += 64) {
        const float v = xr[c];
        const float cm = fmaxf(m, v);
        s = (m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - cm) * kLog2e)) +
            exp_shifted(v, cm);
        m = cm;
      }
    } else {
      for (int c = lane; c < a.C; c += 64) {
        const float v = xr[c];
        const float cm = fmaxf(m, v);
        s = (m == -INFINITY ? 0.0f : s * __builtin_amdgcn_exp2f((m - cm) * kLog2e)) +
            exp_shifted(v, cm);
        m = cm;
      }
    }
    // Merge lanes: global max, then rescale each lane's sum to it.
    const float gm = wave_max(m);
    const float ls = (m == -INFINITY) ? 0.0f : s * __builtin_amdgcn_exp2f((m - gm) * kLog2e);
    const float gs = wave_sum(ls);
    const float safe = fmaxf(gs, 1.0e-7f);
    const float lse = logf(safe);
    // Second pass for the softmax / gradient outputs: the row is read again,
    // in the first pass's form (U float4s per lane in flight, 16-byte
    // stores; the launcher picks VEC only with aligned outputs).
    const int t = a.labels[row];
    const bool bad = t < 0 || t >= a.C;
    auto out_pass = [&](float *orow, bool grad) __attribute__((always_inline)) {
      auto val = [&](float x, int c) __attribute__((always_inline)) {
        const float sm = exp_shifted(x, gm) / safe;
        return grad ? sce_grad(sm, c == t, bad, a.invN) : sm;
      };
      int c0 = 0;
      if constexpr (VEC) {
        const f32x4 *x4 = reinterpret_cast<const f32x4 *>(xr);
        f32x4 *o4 = reinterpret_cast<f32x4 *>(orow);
        const int n4 = a.C >> 2;
        constexpr int U = 8;
        int base = 0;
        for (; base + 64 * U <= n4; base += 64 * U) {
          f32x4 v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(x4 + base + lane + 64 * u);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int c = base + lane + 64 * u;
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = val(v[u][e], 4 * c + e);
            __builtin_nontemporal_store(o, o4 + c);
          }
        }
        for (int c = base + lane; c < n4; c += 64) {
          const f32x4 v = x4[c];
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = val(v[e], 4 * c + e);
          o4[c] = o;
        }
        c0 = n4 << 2;
      }
      for (int c = c0 + lane; c < a.C; c += 64) orow[c] = val(xr[c], c);
    };
    if (a.softmax) out_pass(a.softmax + (int64_t)row * a.ssm, false);
    if (a.grad) out_pass(a.grad + (int64_t)row * a.sg, true);
    if (lane == 0) {
      float lr;
      if (bad) {
        lr = __builtin_nanf("");
      } else {
        const float shifted = xr[t] - gm;
        lr = lse - shifted;
      }
      a.row_loss[row] = lr;
    }
  }

}

// Row held on chip by one 512-thread workgroup (rows of up to
// 2048*(NV + NL) classes): NV 16-byte chunks per thread in registers and, for
// rows past the registers' 2048*NV classes, NL more per thread in LDS,
// loaded there by LDS-DMA (buffer_load ... lds, no VGPRs).  Every logit is
// read from HBM once, and max / sum of exp are exact two-pass reductions
// over the on-chip row (no running rescale).  With NV = 16 (115 VGPRs, 4
// waves per SIMD) and NL = 9 (72 KB of LDS) two rows fit per CU, up to
// 51200 classes (the GPT vocab of 50304 included).  The row's loss goes to
// the workspace for sce_mean_kernel.
constexpr int kRowThreads = 512;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
  // wave64 reduction, then across the 8 waves through LDS.
  v = is_max ? wave_max(v) : wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();  // red[] may still be read by the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

template <int NV, int NL = 0>
__global__ __launch_bounds__(kRowThreads, 4) void sce_row_kernel(SceArgs a) {
  __shared__ float red[kRowThreads / 64];
  __shared__ f32x4 part[NL > 0 ? kRowThreads * NL : 1];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int n4 = a.C >> 2;
  const float *xr = a.logits + (int64_t)row * a.sx;
  const f32x4 *x4 = reinterpret_cast<const f32x4 *>(xr);
  // LDS part: chunk f = 512 NV + tid + 512 j goes to part[tid + 512 j] (a
  // wave's DMA writes 64 consecutive chunks, lane l at l * 16 bytes), issued
  // first; chunks past the row read as zero and are skipped below.
  // The chunk index's j-dependent part is wave-uniform: the bound and the
  // DMA's scalar offset carry it, so no per-j vector value stays live (the
  // compiler had kept nine of them and spilled five to scratch).
  auto in_part = [&](int j) __attribute__((always_inline)) {
    return tid < n4 - kRowThreads * (NV + j);
  };
  if constexpr (NL > 0) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(xr), (short)0, n4 * 16, 0x00020000);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
    for (int j = 0; j < NL; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void *)(part + wave * 64 + kRowThreads * j), 16, (uint32_t)tid * 16u,
          (uint32_t)(kRowThreads * (NV + j)) * 16u, 0, 0);
  }
  f32x4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = tid + kRowThreads * i;
    v[i] = c < n4 ? __builtin_nontemporal_load(x4 + c)
                  : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  // Rows wholly in registers: the label and its logit are loaded behind the
  // row's loads (the fence keeps their waits from being scheduled ahead of
  // them), so that their latencies pass during the reductions instead of
  // after them (config 5: 81.4 -> 80.6 us forward, 188.5 -> 185.5 us fused,
  // the same bits).  With an LDS part the DMA wait (vmcnt 0) would wait for
  // them too, which measured slower; there they are loaded at the end.
  int t = 0;
  bool bad = false;
  float xt = 0.0f;
  if constexpr (NL == 0) {
    __builtin_amdgcn_sched_barrier(0);
    t = a.labels[row];
    bad = t < 0 || t >= a.C;
    if (tid == 0 && !bad) xt = xr[t];
  }
  // the C % 4 tail (at most 3 values) goes to thread 0's spare lane slots
  float tail[3] = {-INFINITY, -INFINITY, -INFINITY};
  if (tid == 0) {
    const int c0 = n4 * 4;
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (c0 + e < a.C) tail[e] = xr[c0 + e];
  }
  float m = fmaxf(fmaxf(tail[0], tail[1]), tail[2]);
#pragma unroll
  for (int i = 0; i < NV; ++i) m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
  if constexpr (NL > 0) {
    // This lane's LDS chunks were written by its own wave's DMA: its own
    // vmcnt wait makes them visible.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < NL; ++j)
      if (in_part(j)) {
        const f32x4 w = part[tid + kRowThreads * j];
        m = fmaxf(m, fmaxf(fmaxf(w.x, w.y), fmaxf(w.z, w.w)));
      }
  }
  const float gm = block_reduce(m, red, true);
  float s = exp_shifted(tail[0], gm) + exp_shifted(tail[1], gm) + exp_shifted(tail[2], gm);
#pragma unroll
  for (int i = 0; i < NV; ++i)
    s += (exp_shifted(v[i].x, gm) + exp_shifted(v[i].y, gm)) +
         (exp_shifted(v[i].z, gm) + exp_shifted(v[i].w, gm));
  if constexpr (NL > 0) {
#pragma unroll
    for (int j = 0; j < NL; ++j)
      if (in_part(j)) {
        const f32x4 w = part[tid + kRowThreads * j];
        s += (exp_shifted(w.x, gm) + exp_shifted(w.y, gm)) +
             (exp_shifted(w.z, gm) + exp_shifted(w.w, gm));
      }
  }
  const float gs = block_reduce(s, red, false);
  const float safe = fmaxf(gs, 1.0e-7f);
  if (a.softmax) {
    float *sr = a.softmax + (int64_t)row * a.ssm;
    f32x4 *s4 = reinterpret_cast<f32x4 *>(sr);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = tid + kRowThreads * i;
      if (c < n4) {
        f32x4 o;
        o.x = exp_shifted(v[i].x, gm) / safe;
        o.y = exp_shifted(v[i].y, gm) / safe;
        o.z = exp_shifted(v[i].z, gm) / safe;
        o.w = exp_shifted(v[i].w, gm) / safe;
        __builtin_nontemporal_store(o, s4 + c);
      }
    }
    if constexpr (NL > 0) {
#pragma unroll
      for (int j = 0; j < NL; ++j)
        if (in_part(j)) {
          const f32x4 w = part[tid + kRowThreads * j];
          f32x4 o;
          o.x = exp_shifted(w.x, gm) / safe;
          o.y = exp_shifted(w.y, gm) / safe;
          o.z = exp_shifted(w.z, gm) / safe;
          o.w = exp_shifted(w.w, gm) / safe;
          __builtin_nontemporal_store(o, s4 + kRowThreads * NV + tid + kRowThreads * j);
        }
    }
    if (tid == 0)
      for (int c = n4 * 4; c < a.C; ++c) sr[c] = exp_shifted(xr[c], gm) / safe;
  }
  if (a.grad) {
    if constexpr (NL > 0) {
      t = a.labels[row];
      bad = t < 0 || t >= a.C;
    }
    float *gr = a.grad + (int64_t)row * a.sg;
    f32x4 *g4 = reinterpret_cast<f32x4 *>(gr);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = tid + kRowThreads * i;
      if (c < n4) {
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = sce_grad(exp_shifted(v[i][e], gm) / safe, 4 * c + e == t, bad, a.invN);
        __builtin_nontemporal_store(o, g4 + c);
      }
    }
    if constexpr (NL > 0) {
#pragma unroll
      for (int j = 0; j < NL; ++j)
        if (in_part(j)) {
          const int c = kRowThreads * NV + tid + kRowThreads * j;
          const f32x4 w = part[tid + kRowThreads * j];
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = sce_grad(exp_shifted(w[e], gm) / safe, 4 * c + e == t, bad, a.invN);
          __builtin_nontemporal_store(o, g4 + c);
        }
    }
    if (tid == 0)
      for (int c = n4 * 4; c < a.C; ++c)
        gr[c] = sce_grad(exp_shifted(xr[c], gm) / safe, c == t, bad, a.invN);
  }
  if (tid == 0) {
    if constexpr (NL > 0) {
      t = a.labels[row];
      bad = t < 0 || t >= a.C;
    }
    float lr;
    if (bad) {
      lr = __builtin_nanf("");
    } else {
      if constexpr (NL > 0) xt = xr[t];
      lr = logf(safe) - (xt - gm);
    }
    a.row_loss[row] = lr;
  }
}

// Mean of the row losses with the order of lowerFullReduceMeanToSCF
// (NovaToLinalg.cpp:1974-2126): 64 contiguous chunks of ceil(R/64), each
// summed sequentially, then the 64 partials sequentially, then / R.  A
// separate launch: stream order makes every row kernel's stores visible
// without the device-scope fences (an L2 write-back and invalidate per
// wave) that a last-workgroup-done scheme would need.
__global__ __launch_bounds__(64) void sce_mean_kernel(const float *row_loss, int rows,
                                                      float *loss) {
  __shared__ float part[64];
  const int per = (rows + 63) / 64;
  const int start = threadIdx.x * per;
  const int end = min(start + per, rows);
  // A chunk's rows go out 64 at a time (a whole chunk of up to 64 rows
  // at once) and are summed in order (a load-add loop waited out one
  // memory latency per row: ~9 us at 4096 rows).  With the losses 16-byte
  // aligned the chunk is read as up to three single rows up to a 16-byte
  // boundary, float4 loads, and up to three single rows at the end: four
  // times fewer load instructions (forward / fused, the same bits:
  // 4096 x 32000 80.6 -> 78.8 / 185.3 -> 184.0 us, 8192 x 50304 243.2 ->
  // 239.8 / 600.5 -> 598.0 us, 100000 x 64 87.1 -> 52.6 us).
  constexpr int kBatch = 64;
  float p = 0.0f;
  if ((reinterpret_cast<uintptr_t>(row_loss) & 15u) == 0) {
    const int a0 = min(end, (start + 3) & ~3);  // first 16-byte boundary
    const int a1 = max(a0, end & ~3);           // last one
    const f32x4 *r4 = reinterpret_cast<const f32x4 *>(row_loss);
    float hd[3], tl[3];
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      hd[e] = start + e < a0 ? row_loss[start + e] : 0.0f;
      tl[e] = a1 + e < end ? row_loss[a1 + e] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (start + e < a0) p = p + hd[e];
    for (int b0 = a0; b0 < a1; b0 += kBatch) {
      f32x4 v[kBatch / 4];
#pragma unroll
      for (int u = 0; u < kBatch / 4; ++u)
        if (b0 + 4 * u < a1) v[u] = r4[(b0 >> 2) + u];
#pragma unroll
      for (int u = 0; u < kBatch / 4; ++u)
        if (b0 + 4 * u < a1) {
          p = p + v[u].x;
          p = p + v[u].y;
          p = p + v[u].z;
          p = p + v[u].w;
        }
    }
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (a1 + e < end) p = p + tl[e];
  } else {
    for (int b0 = start; b0 < end; b0 += kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = b0 + u < end ? row_loss[b0 + u] : 0.0f;
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (b0 + u < end) p = p + v[u];
    }
  }
  part[threadIdx.x] = p;
  __syncthreads();
  if (threadIdx.x == 0) {
    float total = 0.0f;
    for (int i = 0; i < 64; ++i) total = total + part[i];
    loss[0] = total / (float)rows;
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int32_t launch_layer_norm(const LayerNormProblem &p, hipStream_t s) {
  if (p.rows == 0) return NOVA_HIP_SUCCESS;
  // The persistent kernels' row blocks end up to a grid's worth (2048) of
  // rows past the last: rows stay below 2^31 - 2^20 so that this stays in int.
  if (p.rows > 0x7fffffff - (1 << 20) || p.D > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "layer_norm: %lld rows exceed 2^31 - 2^20 or D exceeds 2^31-1",
                (long long)p.rows);
  LnArgs a;
  a.x = p.x;
  a.gamma = p.gamma;
  a.beta = p.beta;
  a.y = p.y;
  a.mean_sum = p.mean_sum;
  a.rstd = p.rstd;
  a.sx = p.sx;
  a.sy = p.sy;
  a.rows = (int)p.rows;
  a.D = (int)p.D;
  a.eps = p.eps;
  a.invD = 1.0f / (float)p.D;
  const unsigned grid = (unsigned)((p.rows + kWaves - 1) / kWaves);
  const bool vec = (p.D % 4 == 0) && (p.sx % 4 == 0) && (p.sy % 4 == 0) &&
                   aligned16(p.x) && aligned16(p.y) && aligned16(p.gamma) &&
                   aligned16(p.beta);
  // Persistent grid for the register kernels: 8 workgroups per CU (2 for
  // the widest rows), never more than one row per wave.  More workgroups
  // than fit at once keep rows queued behind the resident ones: each row's
  // stores wait for all of its loads (the reduction sits between them), and
  // the queued waves cover that gap.  At D = 4096 on MI355X, 8 per CU ran
  // ~2% faster than 4 per CU.
  //
  // Rows of 1025..4096 (16 float4 per lane; 236 VGPRs, two waves per SIMD,
  // two workgroups per CU) instead go three to a workgroup: one row for
  // each of three waves, the fourth only helps stage gamma and beta and
  // exits, so six rows per CU are in flight rather than eight.  HBM serves
  // the row streams better at that depth: at 16384 x 4096, 3 rows per
  // workgroup ran 88.8 us, 2 rows 90.0, 4 rows 96.4, 5 rows 92.3, 8 rows
  // (the persistent grid) 94.4, and one resident workgroup per CU (three
  // rows) 93.9 (in-process A/B, 3 x 300 launches each).
  const unsigned cus = (unsigned)(device_cu_count() > 0 ? device_cu_count() : 256);
  const unsigned pgrid8 = grid < 8u * cus ? grid : 8u * cus;
  const unsigned pgrid2 = grid < 2u * cus ? grid : 2u * cus;
  const unsigned grid3 = (unsigned)((p.rows + 2) / 3);
  if (vec && p.D == 256 * 4)
    hipLaunchKernelGGL((layer_norm_reg_kernel<4, true>), dim3(pgrid8), dim3(256), 0, s, a);
  else if (vec && p.D <= 256 * 4)
    hipLaunchKernelGGL((layer_norm_reg_kernel<4, false>), dim3(pgrid8), dim3(256), 0, s, a);
  else if (vec && p.D == 256 * 16)
    hipLaunchKernelGGL((layer_norm_reg_kernel<16, true>), dim3(grid3), dim3(256), 0, s, a);
  else if (vec && p.D <= 256 * 16)
    hipLaunchKernelGGL((layer_norm_reg_kernel<16, false>), dim3(grid3), dim3(256), 0, s, a);
  else if (vec && p.D <= 256 * 32)
    hipLaunchKernelGGL((layer_norm_reg_kernel<32, false>), dim3(pgrid2), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(layer_norm_any_kernel, dim3(grid), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "layer_norm launch");
}

namespace {
// Row kernels then the mean, with the per-row losses in ws[0, rows).
int32_t launch_sce_into(const SceProblem &p, float *ws, hipStream_t s) {
  SceArgs a;
  a.logits = p.logits;
  a.labels = p.labels;
  a.loss = p.loss;
  a.softmax = p.softmax;
  a.grad = p.grad;
  a.row_loss = ws;
  a.sx = p.sx;
  a.ssm = p.ssm;
  a.sg = p.sg;
  a.invN = p.rows > 0 ? (float)(1.0 / (double)p.rows) : 0.0f;
  a.rows = (int)p.rows;
  a.C = (int)p.C;
  const unsigned grid = (unsigned)((p.rows + kWaves - 1) / kWaves);
  const bool vec = (p.sx % 4 == 0) && aligned16(p.logits) &&
                   (!p.softmax || (p.ssm % 4 == 0 && aligned16(p.softmax))) &&
                   (!p.grad || (p.sg % 4 == 0 && aligned16(p.grad)));
  // Rows of 2K..51200 classes: one workgroup per row, row on chip (in
  // registers, past 32768 classes partly in LDS).
  const int64_t n4 = p.C / 4;
  if (vec && p.rows > 0 && p.C > 2048 && n4 <= (int64_t)kRowThreads * 25) {
    const unsigned g = (unsigned)p.rows;
    if (n4 <= kRowThreads * 4)
      hipLaunchKernelGGL(sce_row_kernel<4>, dim3(g), dim3(kRowThreads), 0, s, a);
    else if (n4 <= kRowThreads * 8)
      hipLaunchKernelGGL(sce_row_kernel<8>, dim3(g), dim3(kRowThreads), 0, s, a);
    else if (n4 <= kRowThreads * 16)
      hipLaunchKernelGGL(sce_row_kernel<16>, dim3(g), dim3(kRowThreads), 0, s, a);
    else
      hipLaunchKernelGGL((sce_row_kernel<16, 9>), dim3(g), dim3(kRowThreads), 0, s, a);
  } else if (vec && p.rows > 0) {
    hipLaunchKernelGGL(sce_kernel<true>, dim3(grid), dim3(256), 0, s, a);
  } else if (p.rows > 0) {
    hipLaunchKernelGGL(sce_kernel<false>, dim3(grid), dim3(256), 0, s, a);
  }
  int32_t rc = check_hip(hipGetLastError(), "sce launch");
  if (rc) return rc;
  // An empty batch still gets the mean: 0 / 0 = NaN, as the reference's
  // division by the element count gives.
  hipLaunchKernelGGL(sce_mean_kernel, dim3(1), dim3(64), 0, s, a.row_loss, a.rows, a.loss);
  return check_hip(hipGetLastError(), "sce mean launch");
}

// Row losses of the entry point that allocates nothing: one array per GPU,
// held until the process ends, shared by every call on that GPU (calls
// that overlap on one GPU race on it).  Every row's loss is written before
// the mean reads it, so nothing needs clearing between calls.  In host
// code `scratch` names a host-side stand-in: kernels get the device
// address from hipGetSymbolAddress, looked up once per device.
constexpr int64_t kScratchRows = SCE_NOALLOC_MAX_ROWS;
static __device__ __align__(256) float scratch[kScratchRows];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices] = {nullptr};

int32_t scratch_of_device(float **out) {
  int dev = -1;
  int32_t rc = check_hip(hipGetDevice(&dev), "sce_noalloc: hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(NOVA_HIP_EDEVICE, "sce_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                   "sce_noalloc: hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    g_scratch_ptr[dev] = static_cast<float *>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return NOVA_HIP_SUCCESS;
}
}  // namespace

int32_t launch_sce(const SceProblem &p, hipStream_t s) {
  // The mean's 64 chunks of ceil(rows / 64) end up to 63 rows past the
  // last, its batches of 64 up to 63 more: rows stay below 2^31 - 2^20.
  if (p.rows > 0x7fffffff - (1 << 20) || p.C > 0x7fffffff)
    return fail(NOVA_HIP_ERANGE, "sce: %lld rows exceed 2^31 - 2^20 or C exceeds 2^31-1",
                (long long)p.rows);
  // Workspace: the per-row losses, held until the mean is enqueued.
  WorkspaceLease lease(s, (size_t)p.rows * 4 + 4);
  float *ws = static_cast<float *>(lease.get());
  if (!ws) return NOVA_HIP_ENOMEM;
  return launch_sce_into(p, ws, s);
}

int32_t launch_sce_noalloc(const SceProblem &p, hipStream_t s) {
  if (p.rows > kScratchRows)
    return fail(NOVA_HIP_ERANGE, "sce_noalloc: %lld rows exceed the scratch maximum of %lld",
                (long long)p.rows, (long long)kScratchRows);
  if (p.C > 0x7fffffff) return fail(NOVA_HIP_ERANGE, "sce: size exceeds 2^31-1");
  float *ws = nullptr;
  int32_t rc = scratch_of_device(&ws);
  if (rc) return rc;
  return launch_sce_into(p, ws, s);
}

}  // namespace nova_hip
