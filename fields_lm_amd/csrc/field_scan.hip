// field_scan.hip — gfx950 kernels and C ABI for the Fields LM Field recurrence.
//
// Path (reference: src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py,
// cited below as "canon"):
//   fused_field_read                      canon:1108-1123  -> fl_scan_forward
//   _field_chunk_summary_kernel           canon:443-516    -> fl_chunk_summary_kernel
//   _field_chunk_carry_kernel             canon:519-550    -> fl_chunk_carry_kernel
//   _field_chunk_materialize_kernel       canon:553-622    -> fl_chunk_materialize_kernel
//   (no reference counterpart)                             -> fl_decode_step_kernel
//
// Work decomposition (MI355X: 64-lane waves, 256 CUs in 8 XCDs, HBM3E):
//   * lane  <-> K adjacent channels, so one wave-wide load of a raw segment is a single
//     64*K-element contiguous run (512 B for bf16 K=4) and one store of a read segment is
//     64*K*4 contiguous bytes;
//   * wave  <-> L consecutive time steps of the chunk, processed sequentially per lane;
//   * block <-> (batch row, channel tile of 64*K channels, time chunk of W*L = kChunkT steps).
// The time-parallel prefix inside a chunk runs across the W waves through LDS (one affine
// summary per wave), the prefix across chunks runs in fl_chunk_carry_kernel.
//
// The affine map of one step is s -> a*s + b with a = (1-v)*lam, b = gamma*v*inj (complex).
// Chunk summaries compose these maps: (A,B) then (a,b) gives (a*A, a*B + b).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "fields_amd.h"

namespace {

constexpr float kVacancyMax = 0.9f;  // canon:68 VAC_MAX
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kChunkT = 64;      // time steps per chunk; every tiling below uses W*L == kChunkT
constexpr int kCarryWaves = 16;  // waves (chunk groups) per block in fl_chunk_carry_kernel

typedef unsigned short bf16_bits;

// ------------------------------------------------------------------------------------------
// element loads: K adjacent channels as fp32
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename RawT, int K>
struct Load;

template <>
struct Load<float, 1> {
  __device__ __forceinline__ static void run(const float* p, float* o) { o[0] = p[0]; }
};
template <>
struct Load<float, 2> {
  __device__ __forceinline__ static void run(const float* p, float* o) {
    float2 v = *reinterpret_cast<const float2*>(p);
    o[0] = v.x; o[1] = v.y;
  }
};
template <>
struct Load<float, 4> {
  __device__ __forceinline__ static void run(const float* p, float* o) {
    float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
};
template <>
struct Load<bf16_bits, 1> {
  __device__ __forceinline__ static void run(const bf16_bits* p, float* o) {
    o[0] = __uint_as_float(static_cast<uint32_t>(p[0]) << 16);
  }
};
template <>
struct Load<bf16_bits, 2> {
  __device__ __forceinline__ static void run(const bf16_bits* p, float* o) {
    uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    o[0] = bf16_lo(w); o[1] = bf16_hi(w);
  }
};
template <>
struct Load<bf16_bits, 4> {
  __device__ __forceinline__ static void run(const bf16_bits* p, float* o) {
    uint2 w = *reinterpret_cast<const uint2*>(p);
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x); o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
  }
};

template <int K>
struct Store;
template <>
struct Store<1> {
  __device__ __forceinline__ static void run(float* p, const float* v) { p[0] = v[0]; }
};
template <>
struct Store<2> {
  __device__ __forceinline__ static void run(float* p, const float* v) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  }
};
template <>
struct Store<4> {
  __device__ __forceinline__ static void run(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// ------------------------------------------------------------------------------------------
// gates (canon:487-505, 599-615): tanh written as 1 - 2/(1+e^{2x}) (= 2*sigmoid(2x) - 1),
// sigmoid as 1/(1+e^{-x}); exp via v_exp_f32 (2^x), reciprocal via v_rcp_f32.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void gates(float zr, float zi, float zv, float gm, float& v,
                                      float& br, float& bi) {
  const float er = __builtin_amdgcn_exp2f(zr * (2.0f * kLog2e));
  const float ei = __builtin_amdgcn_exp2f(zi * (2.0f * kLog2e));
  const float ev = __builtin_amdgcn_exp2f(zv * -kLog2e);
  const float inj_r = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + er);
  const float inj_i = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + ei);
  v = kVacancyMax * __builtin_amdgcn_rcpf(1.0f + ev);
  const float scale = gm * v;
  br = scale * inj_r;
  bi = scale * inj_i;
}

// (A,B) <- step (a,b) applied after (A,B)
__device__ __forceinline__ void compose(float ar, float ai, float br, float bi, float& Ar,
                                        float& Ai, float& Br, float& Bi) {
  const float nAr = ar * Ar - ai * Ai;
  const float nAi = ar * Ai + ai * Ar;
  const float nBr = ar * Br - ai * Bi + br;
  const float nBi = ar * Bi + ai * Br + bi;
  Ar = nAr; Ai = nAi; Br = nBr; Bi = nBi;
}

// ------------------------------------------------------------------------------------------
// Phase 1: per-chunk affine summary (A,B) of kChunkT steps.
// agg layout [B][n_chunks][4][C]: planes Ar, Ai, Br, Bi.
// ------------------------------------------------------------------------------------------
template <typename RawT, int K, int L, int W>
__global__ __launch_bounds__(W * 64) void fl_chunk_summary_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    const float* __restrict__ tr, const float* __restrict__ ti, const float* __restrict__ gamma,
    float* __restrict__ agg) {
  static_assert(W * L == kChunkT, "chunk length mismatch");
  constexpr int CT = 64 * K;
  __shared__ float s_sum[W][4][CT];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int chunk = blockIdx.x;
  const int b = blockIdx.z;
  const int c0 = blockIdx.y * CT + lane * K;
  const bool ok = c0 < C;  // C % K == 0, so all K channels are in range together

  float lr[K], li[K], gm[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    lr[k] = ok ? tr[c0 + k] : 0.f;
    li[k] = ok ? ti[c0 + k] : 0.f;
    gm[k] = ok ? gamma[c0 + k] : 0.f;
  }

  const int t0 = chunk * kChunkT + wave * L;
  const RawT* base = raw + (int64_t)b * sb + c0;
  float z[L][3][K];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int t = t0 + j;
    if (ok && t < T) {
      const RawT* p = base + (int64_t)t * st;
      Load<RawT, K>::run(p, z[j][0]);
      Load<RawT, K>::run(p + C, z[j][1]);
      Load<RawT, K>::run(p + 2 * C, z[j][2]);
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) z[j][0][k] = z[j][1][k] = z[j][2][k] = 0.f;
    }
  }

  float Ar[K], Ai[K], Br[K], Bi[K];
#pragma unroll
  for (int k = 0; k < K; ++k) { Ar[k] = 1.f; Ai[k] = 0.f; Br[k] = 0.f; Bi[k] = 0.f; }
#pragma unroll
  for (int j = 0; j < L; ++j) {
    if (t0 + j < T) {  // steps past T are the identity map (canon:497-501)
#pragma unroll
      for (int k = 0; k < K; ++k) {
        float v, br, bi;
        gates(z[j][0][k], z[j][1][k], z[j][2][k], gm[k], v, br, bi);
        const float keep = 1.f - v;
        compose(keep * lr[k], keep * li[k], br, bi, Ar[k], Ai[k], Br[k], Bi[k]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s_sum[wave][0][lane * K + k] = Ar[k];
    s_sum[wave][1][lane * K + k] = Ai[k];
    s_sum[wave][2][lane * K + k] = Br[k];
    s_sum[wave][3][lane * K + k] = Bi[k];
  }
  __syncthreads();
  if (wave == 0 && ok) {
    // compose the wave summaries in time order
#pragma unroll
    for (int k = 0; k < K; ++k) { Ar[k] = 1.f; Ai[k] = 0.f; Br[k] = 0.f; Bi[k] = 0.f; }
#pragma unroll
    for (int u = 0; u < W; ++u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        compose(s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], s_sum[u][3][x], Ar[k], Ai[k],
                Br[k], Bi[k]);
      }
    }
    float* out = agg + ((int64_t)b * n_chunks + chunk) * 4 * C + c0;
    Store<K>::run(out, Ar);
    Store<K>::run(out + C, Ai);
    Store<K>::run(out + 2 * C, Br);
    Store<K>::run(out + 3 * C, Bi);
  }
}

// ------------------------------------------------------------------------------------------
// Phase 2: exclusive scan of chunk summaries per (b, c): carry[k] = state before chunk k.
// Block = kCarryWaves waves x 64 channels; wave g owns a contiguous group of chunks.
// carry layout [B][n_chunks][2][C]; state_in/state_out [B][2C] planar.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kCarryWaves * 64) void fl_chunk_carry_kernel(
    const float* __restrict__ agg, int C, int n_chunks, const float* __restrict__ state_in,
    float* __restrict__ carry, float* __restrict__ state_out) {
  __shared__ float s_grp[kCarryWaves][4][64];
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool ok = c < C;
  const int per = (n_chunks + kCarryWaves - 1) / kCarryWaves;
  const int k_begin = min(g * per, n_chunks);
  const int k_end = min(k_begin + per, n_chunks);
  const float* ab = agg + (int64_t)b * n_chunks * 4 * C + c;

  float Ar = 1.f, Ai = 0.f, Br = 0.f, Bi = 0.f;
  if (ok) {
    for (int k = k_begin; k < k_end; ++k) {
      const float* p = ab + (int64_t)k * 4 * C;
      compose(p[0], p[C], p[2 * C], p[3 * C], Ar, Ai, Br, Bi);
    }
  }
  s_grp[g][0][lane] = Ar;
  s_grp[g][1][lane] = Ai;
  s_grp[g][2][lane] = Br;
  s_grp[g][3][lane] = Bi;
  __syncthreads();
  if (!ok) return;

  float sr = 0.f, si = 0.f;
  if (state_in != nullptr) {
    sr = state_in[(int64_t)b * 2 * C + c];
    si = state_in[(int64_t)b * 2 * C + C + c];
  }
  for (int u = 0; u < g; ++u) {
    const float ar = s_grp[u][0][lane], ai = s_grp[u][1][lane];
    const float nr = ar * sr - ai * si + s_grp[u][2][lane];
    const float ni = ar * si + ai * sr + s_grp[u][3][lane];
    sr = nr; si = ni;
  }
  float* cb = carry + (int64_t)b * n_chunks * 2 * C + c;
  for (int k = k_begin; k < k_end; ++k) {
    cb[(int64_t)k * 2 * C] = sr;
    cb[(int64_t)k * 2 * C + C] = si;
    const float* p = ab + (int64_t)k * 4 * C;
    const float ar = p[0], ai = p[C];
    const float nr = ar * sr - ai * si + p[2 * C];
    const float ni = ar * si + ai * sr + p[3 * C];
    sr = nr; si = ni;
  }
  if (g == kCarryWaves - 1 && state_out != nullptr) {
    state_out[(int64_t)b * 2 * C + c] = sr;
    state_out[(int64_t)b * 2 * C + C + c] = si;
  }
}

// ------------------------------------------------------------------------------------------
// Phase 3: re-run each chunk from its carry-in and write
// read[b,t,:] = [Re s | Im s | Re disp | Im disp]  (canon:583-621)
// ------------------------------------------------------------------------------------------
template <typename RawT, int K, int L, int W>
__global__ __launch_bounds__(W * 64) void fl_chunk_materialize_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    const float* __restrict__ tr, const float* __restrict__ ti, const float* __restrict__ gamma,
    const float* __restrict__ carry, float* __restrict__ read) {
  static_assert(W * L == kChunkT, "chunk length mismatch");
  constexpr int CT = 64 * K;
  __shared__ float s_sum[W][4][CT];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int chunk = blockIdx.x;
  const int b = blockIdx.z;
  const int c0 = blockIdx.y * CT + lane * K;
  const bool ok = c0 < C;

  float lr[K], li[K], gm[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    lr[k] = ok ? tr[c0 + k] : 0.f;
    li[k] = ok ? ti[c0 + k] : 0.f;
    gm[k] = ok ? gamma[c0 + k] : 0.f;
  }

  const int t0 = chunk * kChunkT + wave * L;
  const RawT* base = raw + (int64_t)b * sb + c0;
  // raw -> (v, b) per step, kept in registers between the summary and the materialisation
  float gv[L][K], gbr[L][K], gbi[L][K];
  {
    float z[L][3][K];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int t = t0 + j;
      if (ok && t < T) {
        const RawT* p = base + (int64_t)t * st;
        Load<RawT, K>::run(p, z[j][0]);
        Load<RawT, K>::run(p + C, z[j][1]);
        Load<RawT, K>::run(p + 2 * C, z[j][2]);
      } else {
#pragma unroll
        for (int k = 0; k < K; ++k) z[j][0][k] = z[j][1][k] = z[j][2][k] = 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
      for (int k = 0; k < K; ++k) gates(z[j][0][k], z[j][1][k], z[j][2][k], gm[k], gv[j][k], gbr[j][k], gbi[j][k]);
    }
  }

  if (W > 1) {
    if (wave < W - 1) {
      float Ar[K], Ai[K], Br[K], Bi[K];
#pragma unroll
      for (int k = 0; k < K; ++k) { Ar[k] = 1.f; Ai[k] = 0.f; Br[k] = 0.f; Bi[k] = 0.f; }
#pragma unroll
      for (int j = 0; j < L; ++j) {
        if (t0 + j < T) {
#pragma unroll
          for (int k = 0; k < K; ++k) {
            const float keep = 1.f - gv[j][k];
            compose(keep * lr[k], keep * li[k], gbr[j][k], gbi[j][k], Ar[k], Ai[k], Br[k], Bi[k]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        s_sum[wave][0][lane * K + k] = Ar[k];
        s_sum[wave][1][lane * K + k] = Ai[k];
        s_sum[wave][2][lane * K + k] = Br[k];
        s_sum[wave][3][lane * K + k] = Bi[k];
      }
    }
    __syncthreads();
  }
  if (!ok) return;

  float sr[K], si[K];
  {
    const float* cp = carry + ((int64_t)b * n_chunks + chunk) * 2 * C + c0;
    Load<float, K>::run(cp, sr);
    Load<float, K>::run(cp + C, si);
  }
  for (int u = 0; u < wave; ++u) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int x = lane * K + k;
      const float ar = s_sum[u][0][x], ai = s_sum[u][1][x];
      const float nr = ar * sr[k] - ai * si[k] + s_sum[u][2][x];
      const float ni = ar * si[k] + ai * sr[k] + s_sum[u][3][x];
      sr[k] = nr; si[k] = ni;
    }
  }

  float* out = read + ((int64_t)b * T + t0) * 4 * C + c0;
#pragma unroll
  for (int j = 0; j < L; ++j) {
    if (t0 + j < T) {
      float dr[K], di[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        // s + disp = lam*s_prev + b, disp = v*lam*s_prev
        const float mr = lr[k] * sr[k] - li[k] * si[k];
        const float mi = lr[k] * si[k] + li[k] * sr[k];
        dr[k] = gv[j][k] * mr;
        di[k] = gv[j][k] * mi;
        sr[k] = mr - dr[k] + gbr[j][k];
        si[k] = mi - di[k] + gbi[j][k];
      }
      float* o = out + (int64_t)j * 4 * C;
      Store<K>::run(o, sr);
      Store<K>::run(o + C, si);
      Store<K>::run(o + 2 * C, dr);
      Store<K>::run(o + 3 * C, di);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Decode: one token per batch row, state updated in place, read_t emitted in the same pass.
// ------------------------------------------------------------------------------------------
template <typename RawT, int K>
__global__ __launch_bounds__(256) void fl_decode_step_kernel(
    const RawT* __restrict__ raw_t, int64_t sb, int B, int C, const float* __restrict__ tr,
    const float* __restrict__ ti, const float* __restrict__ gamma, float* __restrict__ state,
    float* __restrict__ read_t) {
  const int groups = C / K;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * groups) return;
  const int b = (int)(idx / groups);
  const int c0 = (int)(idx - (int64_t)b * groups) * K;

  float zr[K], zi[K], zv[K], lr[K], li[K], gm[K], sr[K], si[K];
  const RawT* p = raw_t + (int64_t)b * sb + c0;
  Load<RawT, K>::run(p, zr);
  Load<RawT, K>::run(p + C, zi);
  Load<RawT, K>::run(p + 2 * C, zv);
  Load<float, K>::run(tr + c0, lr);
  Load<float, K>::run(ti + c0, li);
  Load<float, K>::run(gamma + c0, gm);
  float* s = state + (int64_t)b * 2 * C + c0;
  Load<float, K>::run(s, sr);
  Load<float, K>::run(s + C, si);

  float dr[K], di[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float v, br, bi;
    gates(zr[k], zi[k], zv[k], gm[k], v, br, bi);
    const float mr = lr[k] * sr[k] - li[k] * si[k];
    const float mi = lr[k] * si[k] + li[k] * sr[k];
    dr[k] = v * mr;
    di[k] = v * mi;
    sr[k] = mr - dr[k] + br;
    si[k] = mi - di[k] + bi;
  }
  Store<K>::run(s, sr);
  Store<K>::run(s + C, si);
  float* o = read_t + (int64_t)b * 4 * C + c0;
  Store<K>::run(o, sr);
  Store<K>::run(o + C, si);
  Store<K>::run(o + 2 * C, dr);
  Store<K>::run(o + 3 * C, di);
}

// ------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// widest channel vector K in {4, 2, 1} that every raw/read/state access allows
int pick_k(int raw_dtype, const void* raw, int64_t C, int64_t sb, int64_t st, const void* read,
           const void* state_a, const void* state_b) {
  const size_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  for (int k = 4; k > 1; k /= 2) {
    if (C % k || sb % k || st % k) continue;
    if (!aligned(raw, esz * k) || !aligned(read, 4 * k)) continue;
    if (state_a && !aligned(state_a, 4 * k)) continue;
    if (state_b && !aligned(state_b, 4 * k)) continue;
    return k;
  }
  return 1;
}

inline int hip_status(hipError_t e) { return e == hipSuccess ? FL_OK : FL_ERR_HIP_BASE + (int)e; }

template <typename RawT, int K>
int launch_chunked3(const RawT* raw, int64_t B, int64_t T, int64_t C, int64_t sb, int64_t st,
                    const float* tr, const float* ti, const float* gamma, const float* state_in,
                    float* state_out, float* read, float* agg, float* carry, hipStream_t stream) {
  constexpr int CT = 64 * K;
  const int n_chunks = (int)cdiv(T, kChunkT);
  const dim3 grid((unsigned)n_chunks, (unsigned)cdiv(C, CT), (unsigned)B);
  fl_chunk_summary_kernel<RawT, K, 8, 8><<<grid, 8 * 64, 0, stream>>>(
      raw, sb, st, (int)T, (int)C, n_chunks, tr, ti, gamma, agg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_status(e);
  const dim3 cgrid((unsigned)cdiv(C, 64), (unsigned)B);
  fl_chunk_carry_kernel<<<cgrid, kCarryWaves * 64, 0, stream>>>(agg, (int)C, n_chunks, state_in,
                                                                 carry, state_out);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_status(e);
  fl_chunk_materialize_kernel<RawT, K, 8, 8><<<grid, 8 * 64, 0, stream>>>(
      raw, sb, st, (int)T, (int)C, n_chunks, tr, ti, gamma, carry, read);
  return hip_status(hipGetLastError());
}

template <typename RawT>
int dispatch_chunked3(int k, const void* raw, int64_t B, int64_t T, int64_t C, int64_t sb,
                      int64_t st, const float* tr, const float* ti, const float* gamma,
                      const float* state_in, float* state_out, float* read, float* agg,
                      float* carry, hipStream_t stream) {
  const RawT* r = static_cast<const RawT*>(raw);
  switch (k) {
    case 4:
      return launch_chunked3<RawT, 4>(r, B, T, C, sb, st, tr, ti, gamma, state_in, state_out,
                                      read, agg, carry, stream);
    case 2:
      return launch_chunked3<RawT, 2>(r, B, T, C, sb, st, tr, ti, gamma, state_in, state_out,
                                      read, agg, carry, stream);
    default:
      return launch_chunked3<RawT, 1>(r, B, T, C, sb, st, tr, ti, gamma, state_in, state_out,
                                      read, agg, carry, stream);
  }
}

template <typename RawT>
int dispatch_decode(int k, const void* raw_t, int64_t B, int64_t C, int64_t sb, const float* tr,
                    const float* ti, const float* gamma, float* state, float* read_t,
                    hipStream_t stream) {
  const RawT* r = static_cast<const RawT*>(raw_t);
  const int64_t threads = B * (C / k);
  const unsigned blocks = (unsigned)cdiv(threads, 256);
  switch (k) {
    case 4:
      fl_decode_step_kernel<RawT, 4><<<blocks, 256, 0, stream>>>(r, sb, (int)B, (int)C, tr, ti,
                                                                  gamma, state, read_t);
      break;
    case 2:
      fl_decode_step_kernel<RawT, 2><<<blocks, 256, 0, stream>>>(r, sb, (int)B, (int)C, tr, ti,
                                                                  gamma, state, read_t);
      break;
    default:
      fl_decode_step_kernel<RawT, 1><<<blocks, 256, 0, stream>>>(r, sb, (int)B, (int)C, tr, ti,
                                                                  gamma, state, read_t);
      break;
  }
  return hip_status(hipGetLastError());
}

// shape limits of the launch geometry: grid.y = C/(64K) and grid.z = B stay <= 65535,
// int32 element counts per row
constexpr int64_t kMaxB = 65535;
constexpr int64_t kMaxC = (int64_t)1 << 20;
constexpr int64_t kMaxT = (int64_t)1 << 30;

size_t workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (B <= 0 || T <= 0 || C <= 0) return 0;
  const int64_t n_chunks = cdiv(T, kChunkT);
  return (size_t)(B * n_chunks * C) * 6 * sizeof(float) + 256;
}

}  // namespace

extern "C" {

const char* fl_version(void) { return "fields_amd 0.1 gfx950"; }

size_t fl_scan_workspace_bytes(int64_t B, int64_t T, int64_t C) { return workspace_bytes(B, T, C); }

int fl_scan_forward_ex(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                       int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                       const float* ti, const float* gamma, const float* state_in,
                       float* state_out, void* read, int read_dtype, void* workspace,
                       size_t workspace_bytes_given, int algo, void* stream) {
  if (raw_dtype != FL_DTYPE_F32 && raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (read_dtype != FL_DTYPE_F32) return FL_ERR_DTYPE;
  if (algo != FL_ALGO_AUTO && algo != FL_ALGO_CHUNKED3) return FL_ERR_INVALID_ARGUMENT;
  if (B <= 0 || T <= 0 || C <= 0 || B > kMaxB || C > kMaxC || T > kMaxT)
    return FL_ERR_INVALID_ARGUMENT;
  if (raw_stride_t < 3 * C || raw_stride_b < 0) return FL_ERR_INVALID_ARGUMENT;
  if (B > 1 && raw_stride_b < (T - 1) * raw_stride_t + 3 * C) return FL_ERR_INVALID_ARGUMENT;
  if (!raw || !tr || !ti || !gamma || !read) return FL_ERR_INVALID_ARGUMENT;
  const size_t need = workspace_bytes(B, T, C);
  if (!workspace || workspace_bytes_given < need) return FL_ERR_WORKSPACE;
  const size_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (!aligned(raw, esz) || !aligned(read, 4) || !aligned(workspace, 16))
    return FL_ERR_INVALID_ARGUMENT;
  if ((state_in && !aligned(state_in, 4)) || (state_out && !aligned(state_out, 4)))
    return FL_ERR_INVALID_ARGUMENT;

  const int k = pick_k(raw_dtype, raw, C, raw_stride_b, raw_stride_t, read, nullptr, nullptr);
  const int64_t n_chunks = cdiv(T, kChunkT);
  float* agg = static_cast<float*>(workspace);
  float* carry = agg + B * n_chunks * 4 * C;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* rd = static_cast<float*>(read);
  if (raw_dtype == FL_DTYPE_BF16)
    return dispatch_chunked3<bf16_bits>(k, raw, B, T, C, raw_stride_b, raw_stride_t, tr, ti,
                                        gamma, state_in, state_out, rd, agg, carry, s);
  return dispatch_chunked3<float>(k, raw, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma,
                                  state_in, state_out, rd, agg, carry, s);
}

int fl_scan_forward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                    int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
                    const float* gamma, const float* state_in, float* state_out, void* read,
                    int read_dtype, void* workspace, size_t workspace_bytes_given, void* stream) {
  return fl_scan_forward_ex(raw, raw_dtype, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma,
                            state_in, state_out, read, read_dtype, workspace,
                            workspace_bytes_given, FL_ALGO_AUTO, stream);
}

int fl_decode_step(const void* raw_t, int raw_dtype, int64_t B, int64_t C, int64_t raw_stride_b,
                   const float* tr, const float* ti, const float* gamma, float* state,
                   void* read_t, int read_dtype, void* stream) {
  if (raw_dtype != FL_DTYPE_F32 && raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (read_dtype != FL_DTYPE_F32) return FL_ERR_DTYPE;
  if (B <= 0 || C <= 0 || B > ((int64_t)1 << 31) / 4 || C > kMaxC) return FL_ERR_INVALID_ARGUMENT;
  if (B * C > ((int64_t)1 << 31)) return FL_ERR_INVALID_ARGUMENT;
  if (raw_stride_b < 3 * C) return FL_ERR_INVALID_ARGUMENT;
  if (!raw_t || !tr || !ti || !gamma || !state || !read_t) return FL_ERR_INVALID_ARGUMENT;
  const size_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (!aligned(raw_t, esz) || !aligned(state, 4) || !aligned(read_t, 4))
    return FL_ERR_INVALID_ARGUMENT;
  int k = pick_k(raw_dtype, raw_t, C, raw_stride_b, 0, read_t, state, nullptr);
  // tr/ti/gamma are read as K-vectors too
  while (k > 1 && !(aligned(tr, 4 * k) && aligned(ti, 4 * k) && aligned(gamma, 4 * k))) k /= 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* rd = static_cast<float*>(read_t);
  if (raw_dtype == FL_DTYPE_BF16)
    return dispatch_decode<bf16_bits>(k, raw_t, B, C, raw_stride_b, tr, ti, gamma, state, rd, s);
  return dispatch_decode<float>(k, raw_t, B, C, raw_stride_b, tr, ti, gamma, state, rd, s);
}

}  // extern "C"
