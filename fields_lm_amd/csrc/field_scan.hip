// field_scan.hip — gfx950 kernels and C ABI for the Fields LM Field recurrence.
//
// Path (reference: src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py,
// cited below as "canon"):
//   fused_field_read                  canon:1108-1123  -> fl_scan_forward
//   _field_chunk_summary_kernel       canon:443-516    -> fl_chunk_summary_kernel / look-back kernel
//   _field_chunk_carry_kernel         canon:519-550    -> fl_chunk_carry_kernel / look-back
//   _field_chunk_materialize_kernel   canon:553-622    -> fl_chunk_materialize_kernel / look-back kernel
//   (no reference counterpart)                         -> fl_decode_step_kernel
//
// Work decomposition (MI355X: 64-lane waves, 256 CUs in 8 XCDs, HBM3E):
//   * lane  <-> K adjacent channels: one wave-wide load of a raw segment is a contiguous run of
//     64*K elements and one store of a read segment is 64*K*4 contiguous bytes;
//   * wave  <-> L consecutive time steps, processed sequentially per lane;
//   * block <-> tile = (batch row, channel tile of 64*K channels, time chunk of W*L steps).
// Raw is read and read is written through buffer instructions whose per-step offset is a
// wave-uniform scalar (the per-lane VGPR offset is just the channel), so the address math costs
// no vector instructions, and whose descriptor bounds make rows past T read as 0 and drop stores.
// For bf16 raw with full channel tiles (the default case) raw and read instead pass through LDS,
// so that every global access is 16 bytes per lane (LDSIO below).
//
// The affine map of one step is s -> a*s + b with a = (1-v)*lam and b = gamma*v*inj (complex).
// Because lam is constant per channel, the map of n full steps is
//   A = lam^n * prod(1 - v)   (a complex constant times a REAL product),   B = state from 0,
// so a summary is (P, B) = (prod(1-v), B) and composing summaries only multiplies by lam^n.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <atomic>
#include <mutex>

#include "fields_amd.h"

// 1: the backward kernel stages its second pass's z_r, z_i in LDS where the layout allows (the
// default); 0 keeps register loads everywhere (a build switch for comparisons)
#ifndef FL_BWD_PREFETCH
#define FL_BWD_PREFETCH 1
#endif

namespace {

constexpr float kVacancyMax = 0.9f;  // canon:68 VAC_MAX
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kChunkT = 64;      // chunk length of the three-phase path
constexpr int kCarryWaves = 16;  // waves (chunk groups) per block in fl_chunk_carry_kernel
constexpr uint32_t kBufDword3 = 0x00020000u;  // gfx9 raw-buffer descriptor word 3

typedef unsigned short bf16_bits;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)kBufDword3);
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ------------------------------------------------------------------------------------------
// element access: K adjacent channels, as fp32
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float raw_value(float x) { return x; }
__device__ __forceinline__ float raw_value(bf16_bits x) { return __uint_as_float((uint32_t)x << 16); }

// raw (and grad_read): buffer load at (voffset, soffset) bytes with cache policy POL
template <typename RawT, int K, int POL = 0>
struct RawLoad;
template <int POL>
struct RawLoad<float, 1, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    o[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, POL));
  }
};
template <int POL>
struct RawLoad<float, 2, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, POL);
    o[0] = __uint_as_float(w.x); o[1] = __uint_as_float(w.y);
  }
};
template <int POL>
struct RawLoad<float, 4, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, POL);
    o[0] = __uint_as_float(w.x); o[1] = __uint_as_float(w.y);
    o[2] = __uint_as_float(w.z); o[3] = __uint_as_float(w.w);
  }
};
template <int POL>
struct RawLoad<bf16_bits, 1, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    o[0] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, POL) << 16);
  }
};
template <int POL>
struct RawLoad<bf16_bits, 2, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, POL);
    o[0] = bf16_lo(w); o[1] = bf16_hi(w);
  }
};
template <int POL>
struct RawLoad<bf16_bits, 4, POL> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, float* o) {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, POL);
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x); o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
  }
};

// read: buffer store of K values as float or as bf16 (round to nearest even, v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t bf16_bits_of(float x) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)x);
}
// Two values rounded to nearest even and packed (lo in bits 15..0): one v_cvt_pk_bf16_f32 with
// both operands, where two scalar conversions compile to two of them, a shift and an OR
// (cold B=8, T=2,048: bf16 read, RMSNorm epilogue). Bit-identical to bf16_bits_of on each half.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  const f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Output stores (read, grad_raw) are streamed: written once, never read back by the kernel. The
// non-temporal hint keeps them from displacing the raw data and the look-back words in the
// caches. With the launch's buffers cold (not resident in the 256 MB Infinity Cache from an
// earlier launch), nt stores beat plain and sc1 stores for every output: B=8, T=2,048, fp32 read
// 43.1 -> 39.3 us, bf16 read 36.2 -> 34.5 us, RMSNorm epilogue 39.1 -> 36.3 us against sc1.
constexpr int kStreamStore = 2;  // buffer store cache policy: nt
// The LDS-staged raw loads are non-temporal too where the output is bf16 (bf16 read, the RMSNorm
// epilogue), and plain where it is fp32. Cold, B=8, T=2,048: bf16 read 32.3 -> 31.6 us, RMSNorm
// epilogue 36.1 -> 34.5 us, B=1, T=65,536: 119.6 -> 117.4 and 150.1 -> 143.0 us; with raw just
// written by a preceding kernel (as the mixer's projection leaves it) unchanged (29.7 -> 30.0,
// 36.9 -> 37.0 us). A copy with the scan's tile pattern and fp32 output runs slower with them
// (35.5 -> 37.0 us). The policy is a constant expression in the kernel itself: passed to the
// load builtin as a call of a constexpr function template, it left the host stubs of those
// kernel instances unemitted (the library then fails to load).
// The backward's grad_read loads (its largest input, read once) are non-temporal: cold, B=8,
// T=2,048 64.9 -> 60.6 us, B=1, T=65,536 235.4 -> 233.0 us; its raw loads stay plain (nt on
// them as well: 61.5 and 230.2 us).
constexpr int kStreamLoad = 2;  // buffer load cache policy: nt

template <typename OutT, int K>
struct ReadStore;
template <>
struct ReadStore<float, 1> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, vo, so, kStreamStore);
  }
};
template <>
struct ReadStore<float, 2> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    u32x2 w;
    w.x = __float_as_uint(v[0]); w.y = __float_as_uint(v[1]);
    __builtin_amdgcn_raw_buffer_store_b64(w, r, vo, so, kStreamStore);
  }
};
template <>
struct ReadStore<float, 4> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    u32x4 w;
    w.x = __float_as_uint(v[0]); w.y = __float_as_uint(v[1]);
    w.z = __float_as_uint(v[2]); w.w = __float_as_uint(v[3]);
    // the whole offset in voffset: a 16-byte store with an SGPR soffset is outside the
    // compiler's wait states for a VALU write of its data VGPRs right after it
    __builtin_amdgcn_raw_buffer_store_b128(w, r, vo + so, 0, kStreamStore);
  }
};
template <>
struct ReadStore<bf16_bits, 1> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)bf16_bits_of(v[0]), r, vo, so, kStreamStore);
  }
};
template <>
struct ReadStore<bf16_bits, 2> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    __builtin_amdgcn_raw_buffer_store_b32(bf16_pair(v[0], v[1]), r, vo, so, kStreamStore);
  }
};
template <>
struct ReadStore<bf16_bits, 4> {
  __device__ __forceinline__ static void run(rsrc_t r, int vo, int so, const float* v) {
    u32x2 w;
    w.x = bf16_pair(v[0], v[1]); w.y = bf16_pair(v[2], v[3]);
    __builtin_amdgcn_raw_buffer_store_b64(w, r, vo, so, kStreamStore);
  }
};

// plain pointer access (decode step, carry planes)
template <typename T, int K>
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
// gates (canon:399-406; the Triton form canon:487-505, 599-615)
//   inj = tanh(zr) + i tanh(zi),   v = 0.9 * sigmoid(zv),   b = gamma * v * inj,
// returned as keep = 1 - v and b. With scale = gamma * v (g9 = 0.9 * gamma per channel):
//   b_r = scale * tanh(zr) = scale - 2 scale / (1 + e^{2 zr})   (one fma after the reciprocal),
//   sigmoid(z) = 1 / (1 + e^{-z}),   keep = 1 - 0.9 sigmoid(zv)   (one fma),
// so a channel-step costs 3 v_exp_f32 (2^x on pre-scaled arguments), 3 v_rcp_f32 and 8
// full-rate ops. Every limit is exact without clamps: e^{2x} = inf gives tanh = 1, e^{2x} = 0
// gives tanh = -1, rcp(inf) = 0 gives sigmoid(-inf) = 0; NaN propagates. Near x = 0 the form
// 1 - 2/(1+e^{2x}) carries an absolute error of a few fp32 ulps of 1 (not relative to tanh x).
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ void gates(float zr, float zi, float zv, float g9, float& keep,
                                      float& br, float& bi) {
  const float er = __builtin_amdgcn_exp2f(zr * (2.0f * kLog2e));
  const float ei = __builtin_amdgcn_exp2f(zi * (2.0f * kLog2e));
  const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zv * -kLog2e));
  const float scale = g9 * sg;
  const float m2 = -2.0f * scale;
  br = fmaf(m2, __builtin_amdgcn_rcpf(1.0f + er), scale);
  bi = fmaf(m2, __builtin_amdgcn_rcpf(1.0f + ei), scale);
  keep = fmaf(-kVacancyMax, sg, 1.0f);
}

// complex power lam^n by repeated squaring (n >= 0)
__device__ __forceinline__ void cpow(float lr, float li, int n, float& pr, float& pi) {
  float rr = 1.f, ri = 0.f, br = lr, bi = li;
  while (n > 0) {
    if (n & 1) {
      const float t = rr * br - ri * bi;
      ri = rr * bi + ri * br;
      rr = t;
    }
    const float t = br * br - bi * bi;
    bi = 2.f * br * bi;
    br = t;
    n >>= 1;
  }
  pr = rr; pi = ri;
}

// s <- A s + B with A = lamn * P (lamn complex, P real)
// Complex product with its rounding written out (real = fma(ar, br, -(ai bi)), imag =
// fma(ar, bi, ai br)): left to -ffp-contract=fast, the contraction of such expressions can differ
// between template instances of one kernel, so their results would not match bit for bit.
__device__ __forceinline__ void cmul(float ar, float ai, float br, float bi, float& re, float& im) {
  re = fmaf(ar, br, -(ai * bi));
  im = fmaf(ar, bi, ai * br);
}

// s <- P * (lam^n s) + B: applies a summary (P, B) of n steps to the state s. The look-back's
// carry equals a predecessor's published inclusive state bit for bit only because both are formed
// by this function with this rounding (cmul, then fma), at whichever call site.
__device__ __forceinline__ void apply_map(float lnr, float lni, float P, float Br, float Bi,
                                          float& sr, float& si) {
  float mr, mi;
  cmul(lnr, lni, sr, si, mr, mi);
  sr = fmaf(P, mr, Br);
  si = fmaf(P, mi, Bi);
}

// ------------------------------------------------------------------------------------------
// wave tile: L steps x K channels per lane
// ------------------------------------------------------------------------------------------
template <typename RawT, int K, int L>
struct WaveTile {
  // gates, kept between summary and materialisation: keep = 1 - v, b
  float gk[L][K], gbr[L][K], gbi[L][K];

  // Loads L rows from the raw descriptor (row j at soffset so0 + j*row_bytes) and forms gates.
  // Rows past the descriptor's bound read as 0; their gates are never used.
  __device__ __forceinline__ void load(rsrc_t r, int vo, int so0, int row_bytes, int plane_bytes,
                                       const float* gm) {
    float z[L][3][K], g9[K];
#pragma unroll
    for (int k = 0; k < K; ++k) g9[k] = kVacancyMax * gm[k];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int so = so0 + j * row_bytes;
      RawLoad<RawT, K>::run(r, vo, so, z[j][0]);
      RawLoad<RawT, K>::run(r, vo, so + plane_bytes, z[j][1]);
      RawLoad<RawT, K>::run(r, vo, so + 2 * plane_bytes, z[j][2]);
    }
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
      for (int k = 0; k < K; ++k)
        gates(z[j][0][k], z[j][1][k], z[j][2][k], g9[k], gk[j][k], gbr[j][k], gbi[j][k]);
    }
  }

  // Gates from bf16 raw staged in LDS: plane p of this wave's row j at s[p*plane + j*64 + lane].
  __device__ __forceinline__ void load_lds(const bf16_bits* s, int plane, int lane,
                                           const float* gm) {
    static_assert(K == 1, "LDS staging holds one channel per lane");
    const float g9 = kVacancyMax * gm[0];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const float zr = __uint_as_float((uint32_t)s[j * 64 + lane] << 16);
      const float zi = __uint_as_float((uint32_t)s[plane + j * 64 + lane] << 16);
      const float zv = __uint_as_float((uint32_t)s[2 * plane + j * 64 + lane] << 16);
      gates(zr, zi, zv, g9, gk[j][0], gbr[j][0], gbi[j][0]);
    }
  }

  // One step from (sr, si) with row j's gates: m = lam * s_prev, disp = v * m = m - keep * m,
  // s = keep * m + b (canon:583-621). The complex product goes through cmul, so that every pass
  // (plain stores, LDS-staged stores, the RMSNorm epilogue's value pass) rounds alike.
  __device__ __forceinline__ void step(int j, int k, float lr, float li, float& sr, float& si,
                                       float& dr, float& di) const {
    float mr, mi;
    cmul(lr, li, sr, si, mr, mi);
    dr = fmaf(-gk[j][k], mr, mr);
    di = fmaf(-gk[j][k], mi, mi);
    sr = fmaf(gk[j][k], mr, gbr[j][k]);
    si = fmaf(gk[j][k], mi, gbi[j][k]);
  }

  // Stores of a per-wave LDS region `stage` (4 planes x R rows x 64 floats, written one channel
  // per lane): read back as 16 bytes of output per lane (4 fp32 or 8 bf16 channels of one
  // row-plane) and stored with 16-byte buffer stores at byte offset off0 + row * row_bytes +
  // plane * plane_bytes + 16 * piece. The whole offset is in voffset, so rows past the
  // descriptor's bound (past T) are dropped by it.
  template <typename OutT, int R>
  __device__ __forceinline__ static void store_stage(rsrc_t w, int lane, int off0, int row_bytes,
                                                     int plane_bytes, const float* stage) {
    // soffset stays the constant 0: a 16-byte store with an SGPR soffset is not covered by
    // the compiler's wait states for a VALU op overwriting the store's data VGPRs right after
    // it, and on gfx950 that overwrite reached memory (component 1, the next instruction's
    // target) for some lanes; with a constant soffset the wait states are inserted
    if constexpr (sizeof(OutT) == 4) {
      // row-plane rp = 4 * i + lane / 16 of instruction i, channels 4 * (lane % 16) .. + 3
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int rp = 4 * i + (lane >> 4), plane = rp / R, row = rp % R, piece = lane & 15;
        const float4 v = *reinterpret_cast<const float4*>(stage + rp * 64 + 4 * piece);
        u32x4 q;
        q.x = __float_as_uint(v.x); q.y = __float_as_uint(v.y);
        q.z = __float_as_uint(v.z); q.w = __float_as_uint(v.w);
        const int off = off0 + 16 * piece + row * row_bytes + plane * plane_bytes;
        __builtin_amdgcn_raw_buffer_store_b128(q, w, off, 0, kStreamStore);
      }
    } else {
      // row-plane rp = 8 * i + lane / 8 of instruction i, channels 8 * (lane % 8) .. + 7
#pragma unroll
      for (int i = 0; i < R / 2; ++i) {
        const int rp = 8 * i + (lane >> 3), plane = rp / R, row = rp % R, piece = lane & 7;
        const float4 a = *reinterpret_cast<const float4*>(stage + rp * 64 + 8 * piece);
        const float4 c = *reinterpret_cast<const float4*>(stage + rp * 64 + 8 * piece + 4);
        u32x4 q;
        q.x = bf16_pair(a.x, a.y); q.y = bf16_pair(a.z, a.w);
        q.z = bf16_pair(c.x, c.y); q.w = bf16_pair(c.z, c.w);
        const int off = off0 + 16 * piece + row * row_bytes + plane * plane_bytes;
        __builtin_amdgcn_raw_buffer_store_b128(q, w, off, 0, kStreamStore);
      }
    }
  }

  // materialize() through a per-wave LDS region `stage` (4 planes x R rows x 64 floats): each
  // group of R rows is written to LDS one channel per lane and stored by store_stage. The tile's
  // 64 channels must all lie below C.
  static constexpr int kStageRows = L >= 16 ? 4 : 2;  // R
  template <typename OutT, int R = kStageRows>
  __device__ __forceinline__ void materialize_lds(rsrc_t w, int lane, int so0, int row_bytes,
                                                  int plane_bytes, int ch_bytes0, int n,
                                                  float* stage, const float* lr, const float* li,
                                                  float* sr, float* si) const {
    static_assert(K == 1 && L % R == 0 && R % 2 == 0, "LDS-staged stores: one channel per lane, whole groups");
#pragma unroll
    for (int g = 0; g < L / R; ++g) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = R * g + r;
        float o[4] = {sr[0], si[0], 0.f, 0.f};
        step(j, 0, lr[0], li[0], o[0], o[1], o[2], o[3]);
        if (j < n) {  // rows from n on lie past T: their stores are dropped, the state stops here
          sr[0] = o[0];
          si[0] = o[1];
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) stage[(p * R + r) * 64 + lane] = o[p];
      }
      store_stage<OutT, R>(w, lane, so0 + R * g * row_bytes + ch_bytes0, row_bytes, plane_bytes, stage);
    }
  }

  // RMSNorm epilogue (K = 1), value pass over rows j0 .. j0 + H - 1: the four read values
  // (Re s, Im s, Re disp, Im disp) of each row from (sr, si), kept in v for the stores, and each
  // row's sum of their squares in ss (0 for lanes outside the channel range, ok false). Rows from
  // n on lie past T: the pass runs through them with no row check (from zero input; their values
  // and sums are never stored or published), and on return (sr, si) is the state after row n - 1,
  // read back from v where the tile is partial (n is wave-uniform, j0 < n <= j0 + H).
  template <int H>
  __device__ __forceinline__ void norm_values(int j0, int n, bool ok, float lr, float li, float& sr,
                                              float& si, float (&v)[L][4], float (&ss)[H]) const {
    static_assert(K == 1, "the RMSNorm epilogue runs one channel per lane");
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const int j = j0 + i;
      v[j][0] = sr;
      v[j][1] = si;
      step(j, 0, lr, li, v[j][0], v[j][1], v[j][2], v[j][3]);
      sr = v[j][0];
      si = v[j][1];
      float acc = v[j][0] * v[j][0];
      acc = fmaf(v[j][1], v[j][1], acc);
      acc = fmaf(v[j][2], v[j][2], acc);
      acc = fmaf(v[j][3], v[j][3], acc);
      ss[i] = ok ? acc : 0.f;
    }
    if (n < j0 + H) {
#pragma unroll
      for (int i = 0; i < H; ++i) {
        if (j0 + i == n - 1) {
          sr = v[j0 + i][0];
          si = v[j0 + i][1];
        }
      }
    }
  }

  // RMSNorm epilogue, stores of rows j0 .. j0 + H - 1 through LDS: row j stores
  // (v[j][p] * scale_j) * nw[p], scale_j taken from lane j - j0 of `scale`, in groups of R rows
  // by store_stage (the tile's 64 channels must all lie below C).
  template <typename OutT, int H, int R = kStageRows>
  __device__ __forceinline__ static void store_norm_lds(rsrc_t w, int lane, int j0, int so0,
                                                        int row_bytes, int plane_bytes,
                                                        int ch_bytes0, float* stage,
                                                        const float (&v)[L][4], float scale,
                                                        const float (&nw)[4]) {
    static_assert(H % R == 0 && R % 2 == 0, "LDS-staged stores: whole groups");
#pragma unroll
    for (int g = 0; g < H / R; ++g) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = R * g + r;
        const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scale), i));
#pragma unroll
        for (int p = 0; p < 4; ++p) stage[(p * R + r) * 64 + lane] = (v[j0 + i][p] * sc) * nw[p];
      }
      store_stage<OutT, R>(w, lane, so0 + (j0 + R * g) * row_bytes + ch_bytes0, row_bytes,
                           plane_bytes, stage);
    }
  }

  // RMSNorm epilogue, register stores of rows j0 .. j0 + H - 1: row j < n stores
  // (v[j][p] * scale_j) * nw[p] from lanes with ok set.
  template <typename OutT, int H>
  __device__ __forceinline__ static void store_norm(rsrc_t w, int vo, int j0, int so0, int row_bytes,
                                                    int plane_bytes, int n, bool ok,
                                                    const float (&v)[L][4], float scale,
                                                    const float (&nw)[4]) {
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const int j = j0 + i;
      const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scale), i));
      if (ok && j < n) {
        const int so = so0 + j * row_bytes;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float o = (v[j][p] * sc) * nw[p];
          ReadStore<OutT, 1>::run(w, vo, so + p * plane_bytes, &o);
        }
      }
    }
  }

  // Summary over all L steps: P = prod(1-v), B = state reached from 0.
  __device__ __forceinline__ void summary(const float* lr, const float* li, float* P, float* Br,
                                          float* Bi) const {
#pragma unroll
    for (int k = 0; k < K; ++k) { P[k] = 1.f; Br[k] = 0.f; Bi[k] = 0.f; }
#pragma unroll
    for (int j = 0; j < L; ++j) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const float keep = gk[j][k];
        const float mr = lr[k] * Br[k] - li[k] * Bi[k];
        const float mi = lr[k] * Bi[k] + li[k] * Br[k];
        Br[k] = fmaf(keep, mr, gbr[j][k]);
        Bi[k] = fmaf(keep, mi, gbi[j][k]);
        P[k] *= keep;
      }
    }
  }

  // Recurrence from (sr, si) over the first n steps, storing
  // read[b,t,:] = [Re s | Im s | Re disp | Im disp] (canon:583-621), row j at so0 + j*row_bytes.
  template <typename OutT>
  __device__ __forceinline__ void materialize(rsrc_t w, int vo, int so0, int row_bytes,
                                              int plane_bytes, int n, const float* lr,
                                              const float* li, float* sr, float* si) const {
#pragma unroll
    for (int j = 0; j < L; ++j) {
      if (j < n) {
        float dr[K], di[K];
#pragma unroll
        for (int k = 0; k < K; ++k) step(j, k, lr[k], li[k], sr[k], si[k], dr[k], di[k]);
        const int so = so0 + j * row_bytes;
        ReadStore<OutT, K>::run(w, vo, so, sr);
        ReadStore<OutT, K>::run(w, vo, so + plane_bytes, si);
        ReadStore<OutT, K>::run(w, vo, so + 2 * plane_bytes, dr);
        ReadStore<OutT, K>::run(w, vo, so + 3 * plane_bytes, di);
      }
    }
  }
};

// Row sums across a wave through LDS (L = 16): v[j] per lane in; on return lane l holds the sum
// over all 64 lanes of v[l / 4] (the four lanes 4r .. 4r + 3 hold row r's sum). buf: 1024 floats
// of LDS owned by this wave. Each lane writes its 16 values as one column, reads 16 consecutive
// values of one row (a quarter of the 64 lanes) and adds them, and two quad exchanges finish the
// row. Every wave adds in the same order. About 20 VALU instructions against about 50 for a
// shuffle butterfly over the 64 lanes (halving exchanges, then xor stages): cold B=8, T=2,048
// RMSNorm epilogue 34.75-35.02 -> 34.59-34.84 us, B=1, T=65,536 143.1-143.6 -> 141.5-142.5 us.
__device__ __forceinline__ float wave_row_sums_lds(const float (&v)[16], int lane, float* buf) {
#pragma unroll
  for (int j = 0; j < 16; ++j) buf[j * 64 + lane] = v[j];
  __builtin_amdgcn_wave_barrier();
  const float4* src = reinterpret_cast<const float4*>(buf + (lane >> 2) * 64 + (lane & 3) * 16);
  const float4 a = src[0], b = src[1], c = src[2], d = src[3];
  float t = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
  t += ((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w));
  t += __shfl_xor(t, 1);
  t += __shfl_xor(t, 2);
  return t;
}

template <int K>
__device__ __forceinline__ void load_params(const float* __restrict__ tr, const float* __restrict__ ti,
                                            const float* __restrict__ gamma, int c0, bool ok,
                                            float* lr, float* li, float* gm) {
#pragma unroll
  for (int k = 0; k < K; ++k) {
    lr[k] = ok ? tr[c0 + k] : 0.f;
    li[k] = ok ? ti[c0 + k] : 0.f;
    gm[k] = ok ? gamma[c0 + k] : 0.f;
  }
}

// Buffer descriptors of one tile: raw from row t_begin of batch row b to the end of the tile's
// last row (row min(t_begin + span, T) - 1), read over the same rows. Covering only the tile's
// rows keeps every descriptor below 2 GiB whatever T is (a row is below 4 MiB, a tile at most
// 128 rows), and rows past T still read as 0 and drop their stores.
struct TileIo {
  rsrc_t raw, read;
  int vo_raw, vo_read;          // per-lane channel byte offsets
  int raw_row, raw_plane;       // bytes between rows / between the 3 raw planes
  int read_row, read_plane;     // bytes between rows / between the 4 read planes
};

template <typename RawT, typename OutT>
__device__ __forceinline__ TileIo tile_io(const RawT* raw, int64_t sb, int64_t st, OutT* read,
                                          int T, int C, int b, int t_begin, int span, int c0) {
  TileIo io;
  const int rows = min(T - t_begin, span);  // >= 1
  const RawT* rbase = raw + (int64_t)b * sb + (int64_t)t_begin * st;
  io.raw = make_rsrc(rbase, (uint32_t)(((int64_t)(rows - 1) * st + 3 * (int64_t)C) * sizeof(RawT)));
  OutT* wbase = read + ((int64_t)b * T + t_begin) * 4 * C;
  io.read = make_rsrc(wbase, (uint32_t)((int64_t)rows * 4 * C * sizeof(OutT)));
  io.vo_raw = c0 * (int)sizeof(RawT);
  io.vo_read = c0 * (int)sizeof(OutT);
  io.raw_row = (int)(st * (int64_t)sizeof(RawT));
  io.raw_plane = C * (int)sizeof(RawT);
  io.read_row = 4 * C * (int)sizeof(OutT);
  io.read_plane = C * (int)sizeof(OutT);
  return io;
}

// ------------------------------------------------------------------------------------------
// Three-phase path (FL_ALGO_CHUNKED3), chunks of kChunkT = W*L steps.
// Phase 1: per-chunk summary (P, B). agg layout [B][n_chunks][3][C]: P, Br, Bi. The last
// chunk's summary is never consumed and is not computed.
// ------------------------------------------------------------------------------------------
template <typename RawT, int K, int L, int W>
__global__ __launch_bounds__(W * 64) void fl_chunk_summary_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    const float* __restrict__ tr, const float* __restrict__ ti, const float* __restrict__ gamma,
    float* __restrict__ agg) {
  static_assert(W * L == kChunkT, "chunk length mismatch");
  constexpr int CT = 64 * K;
  __shared__ float s_sum[W][3][CT];

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  if (chunk == n_chunks - 1) return;
  const int b = blockIdx.z;
  const int c0 = blockIdx.y * CT + lane * K;
  const bool ok = c0 < C;  // C % K == 0, so all K channels are in range together

  float lr[K], li[K], gm[K];
  load_params<K>(tr, ti, gamma, c0, ok, lr, li, gm);
  const TileIo io = tile_io<RawT, float>(raw, sb, st, nullptr, T, C, b, chunk * kChunkT, kChunkT, c0);
  WaveTile<RawT, K, L> tile;
  tile.load(io.raw, io.vo_raw, wave * L * io.raw_row, io.raw_row, io.raw_plane, gm);
  float P[K], Br[K], Bi[K];
  tile.summary(lr, li, P, Br, Bi);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s_sum[wave][0][lane * K + k] = P[k];
    s_sum[wave][1][lane * K + k] = Br[k];
    s_sum[wave][2][lane * K + k] = Bi[k];
  }
  __syncthreads();
  if (wave == 0 && ok) {
    float lLr[K], lLi[K];
#pragma unroll
    for (int k = 0; k < K; ++k) cpow(lr[k], li[k], L, lLr[k], lLi[k]);
#pragma unroll
    for (int k = 0; k < K; ++k) { P[k] = 1.f; Br[k] = 0.f; Bi[k] = 0.f; }
    for (int u = 0; u < W; ++u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        apply_map(lLr[k], lLi[k], s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], Br[k], Bi[k]);
        P[k] *= s_sum[u][0][x];
      }
    }
    float* out = agg + ((int64_t)b * n_chunks + chunk) * 3 * C + c0;
    Store<K>::run(out, P);
    Store<K>::run(out + C, Br);
    Store<K>::run(out + 2 * C, Bi);
  }
}

// Phase 2: exclusive scan of chunk summaries per (b, c): carry[k] = state before chunk k.
// Block = kCarryWaves waves x 64 channels; wave g owns a contiguous group of chunks.
// carry layout [B][n_chunks][2][C]. Only chunks 0..n_chunks-2 have summaries.
__global__ __launch_bounds__(kCarryWaves * 64) void fl_chunk_carry_kernel(
    const float* __restrict__ agg, int C, int n_chunks, const float* __restrict__ tr,
    const float* __restrict__ ti, const float* __restrict__ state_in, float* __restrict__ carry) {
  __shared__ float s_grp[kCarryWaves][4][64];
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool ok = c < C;
  const int n_sum = n_chunks - 1;  // summaries that exist
  const int per = (n_sum + kCarryWaves - 1) / kCarryWaves;
  const int k_begin = min(g * per, n_sum);
  const int k_end = min(k_begin + per, n_sum);
  const float* ab = agg + (int64_t)b * n_chunks * 3 * C + c;
  float lcr = 1.f, lci = 0.f;  // lam^kChunkT
  if (ok) cpow(tr[c], ti[c], kChunkT, lcr, lci);

  // group map as (A complex, B complex)
  float Ar = 1.f, Ai = 0.f, Br = 0.f, Bi = 0.f;
  if (ok) {
    for (int k = k_begin; k < k_end; ++k) {
      const float* p = ab + (int64_t)k * 3 * C;
      const float P = p[0];
      const float ar = P * lcr, ai = P * lci;
      const float nAr = ar * Ar - ai * Ai;
      const float nAi = ar * Ai + ai * Ar;
      const float nBr = ar * Br - ai * Bi + p[C];
      const float nBi = ar * Bi + ai * Br + p[2 * C];
      Ar = nAr; Ai = nAi; Br = nBr; Bi = nBi;
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
    const float* p = ab + (int64_t)k * 3 * C;
    apply_map(lcr, lci, p[0], p[C], p[2 * C], sr, si);
  }
  if (g == kCarryWaves - 1) {  // the state entering the last chunk
    cb[(int64_t)n_sum * 2 * C] = sr;
    cb[(int64_t)n_sum * 2 * C + C] = si;
  }
}

// Phase 3: re-run each chunk from its carry-in and write read (and state_out).
template <typename RawT, typename OutT, int K, int L, int W>
__global__ __launch_bounds__(W * 64) void fl_chunk_materialize_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    const float* __restrict__ tr, const float* __restrict__ ti, const float* __restrict__ gamma,
    const float* __restrict__ carry, OutT* __restrict__ read, float* __restrict__ state_out) {
  static_assert(W * L == kChunkT, "chunk length mismatch");
  constexpr int CT = 64 * K;
  __shared__ float s_sum[W][3][CT];

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int chunk = blockIdx.x;
  const int b = blockIdx.z;
  const int c0 = blockIdx.y * CT + lane * K;
  const bool ok = c0 < C;

  float lr[K], li[K], gm[K];
  load_params<K>(tr, ti, gamma, c0, ok, lr, li, gm);
  const int t_begin = chunk * kChunkT;
  const TileIo io = tile_io<RawT, OutT>(raw, sb, st, read, T, C, b, t_begin, kChunkT, c0);
  WaveTile<RawT, K, L> tile;
  tile.load(io.raw, io.vo_raw, wave * L * io.raw_row, io.raw_row, io.raw_plane, gm);
  const int n = min(max(T - (t_begin + wave * L), 0), L);  // valid steps of this wave
  if (W > 1) {
    if (wave < W - 1) {
      // read only by later waves, which have valid steps only if this wave is full
      float P[K], Br[K], Bi[K];
      tile.summary(lr, li, P, Br, Bi);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        s_sum[wave][0][lane * K + k] = P[k];
        s_sum[wave][1][lane * K + k] = Br[k];
        s_sum[wave][2][lane * K + k] = Bi[k];
      }
    }
    __syncthreads();
  }
  if (!ok || n == 0) return;
  float sr[K], si[K];
  {
    const float* cp = carry + ((int64_t)b * n_chunks + chunk) * 2 * C + c0;
    Load<float, K>::run(cp, sr);
    Load<float, K>::run(cp + C, si);
  }
  if (wave > 0) {
    float lLr[K], lLi[K];
#pragma unroll
    for (int k = 0; k < K; ++k) cpow(lr[k], li[k], L, lLr[k], lLi[k]);
    for (int u = 0; u < wave; ++u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        apply_map(lLr[k], lLi[k], s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], sr[k], si[k]);
      }
    }
  }
  tile.template materialize<OutT>(io.read, io.vo_read, wave * L * io.read_row, io.read_row,
                                 io.read_plane, n, lr, li, sr, si);
  if (state_out != nullptr && t_begin + wave * L + n == T) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      state_out[(int64_t)b * 2 * C + c0 + k] = sr[k];
      state_out[(int64_t)b * 2 * C + C + c0 + k] = si[k];
    }
  }
}

// ------------------------------------------------------------------------------------------
// Single-pass path (FL_ALGO_LOOKBACK): one launch, raw read once, read written once.
//
// Tiles = (chain = (b, channel tile), chunk of W*L steps); ticket -> tile is chunk-major, so the
// predecessors of ticket t in its chain are t - n_chains, t - 2*n_chains, ... and a tile only
// waits on lower tickets. Tickets come either in block order (block i takes ticket i; the host's
// choice for short chains) or from one atomic counter, in the order blocks start. From the
// counter, a ticket's predecessors were taken earlier by blocks that are already running, whatever
// the dispatch order. In block order, progress rests on the dispatcher issuing each XCD's share of
// the grid in block order: every block resident ahead of the lowest unfinished tile on its XCD has
// a lower index, so that tile is always resident. A tile
//   1. loads its raw tile into registers and forms the gates;
//   2. composes its summary (P, B) and publishes it (status AGG);
//   3. looks back over its chain for the nearest tile with a published inclusive state (status
//      INCL); the summaries of the tiles after it are fetched by all W waves in parallel and
//      applied to it one by one, which gives the carry-in (the same values whichever tile's
//      inclusive state was found: see lookback_carry);
//   4. publishes its inclusive state (status INCL) and materialises.
// With the RMSNorm epilogue (NORM), step 4 first runs the tile's recurrence once more without
// storing, to form each row's partial sum of squares over the tile's channels; publishes the
// partials (one word per row and channel tile); waits for the partials of the other channel
// tiles of the same (batch row, chunk) — the n_ctiles consecutive tickets of its group, the
// lowest incomplete group always resident by the same arguments, none of them waiting on this
// block — and
// stores read * rsqrt(mean(read^2) + eps) * weight. The inclusive state is published before
// that wait, so the chain's successors never wait on the exchange.
// Every published value is a 64-bit word (value | tag), tag = epoch<<2 | kind, written and
// read with relaxed agent-scope atomics (device-coherent across XCD L2s). A reader checks
// each word's own tag, so no fences are needed, and the epoch (bumped by the last block of
// every launch) makes words of earlier launches stale without clearing the workspace.
// Waits sleep between polls and give up after the header's spin limit (2^20 polls unless set),
// so every wave terminates. A wait that gives up sets the error word (and the host-visible word,
// when the header names one) and poisons what depends on it with NaN: the tile's carry (and so
// its outputs and every later tile of its chain), its RMSNorm scale, or the parameter-gradient
// sums, so that a result computed without a value it needed cannot pass for a valid one.
// ------------------------------------------------------------------------------------------
// Every word sits in its own 128-byte line: the ticket counter is hammered by the blocks' first
// atomic (long chains), `done` by their last one.
struct LookbackHeader {
  unsigned int done;   // tiles finished in this launch (blocks that refused a ticket included)
  unsigned int pad0[31];
  unsigned int error;  // bit 0: a wait gave up; bit 1: ticket out of range
  unsigned int pad1[31];
  // bits 63..32 launch epoch, bits 31..0 tickets taken in this launch (block-order launches
  // only read the epoch)
  unsigned long long ticket;
  unsigned long long pad2[15];
  unsigned int spin_limit;        // polls before a wait gives up; 0: kSpinLimit (set by the caller)
  unsigned int pad3;
  unsigned long long host_error;  // address of a host-visible u32 also set on error; 0: none
  unsigned long long pad4[14];
};

constexpr uint32_t kTagAgg = 1u;
constexpr uint32_t kTagIncl = 2u;
constexpr uint32_t kTagSib = 3u;   // per-row partial sum of squares (NORM epilogue)
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr size_t kHeaderBytes = 2048;
static_assert(sizeof(LookbackHeader) <= kHeaderBytes, "header region too small");
static_assert(offsetof(LookbackHeader, error) == 128 && offsetof(LookbackHeader, ticket) == 256 &&
                  offsetof(LookbackHeader, spin_limit) == 384 &&
                  offsetof(LookbackHeader, host_error) == 392,
              "header offsets are part of the C ABI");

__device__ __forceinline__ uint32_t spin_limit_of(const LookbackHeader* hdr) {
  const uint32_t l = __hip_atomic_load(&hdr->spin_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return l != 0u ? l : kSpinLimit;
}

// Sets `bits` in the header's error word and, when the header names one, in the host-visible
// word (a plain store: the host only tests it for non-zero).
__device__ __forceinline__ void report_error(LookbackHeader* hdr, uint32_t bits) {
  atomicOr(&hdr->error, bits);
  const unsigned long long h =
      __hip_atomic_load(&hdr->host_error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // through a global-address-space pointer: a store through a generic pointer may write LDS as
  // far as the compiler knows, and would make every later LDS access of the kernel wait for all
  // outstanding global loads and stores
  if (h != 0ull)
    __hip_atomic_store(reinterpret_cast<__attribute__((address_space(1))) uint32_t*>(h), bits,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ float poison() { return __builtin_nanf(""); }

// The counter armed for the next launch (next epoch), by the launch's last block.
__device__ __forceinline__ void rearm(LookbackHeader* hdr, uint32_t epoch) {
  const unsigned long long armed = (unsigned long long)(epoch + 1u) << 32;
  __hip_atomic_store(&hdr->ticket, armed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&hdr->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// One thread's count of its block toward the launch's end; the last block re-arms the counter.
// Blocks that refused an out-of-range ticket count too, so a counter that was out of range is
// re-armed by the launch that saw it. (The backward scan ends every block here: its reduction
// launch, which runs after it, clears the workspace at the epoch wrap.)
__device__ __forceinline__ void finish_block(LookbackHeader* hdr, uint32_t n_tiles, uint32_t epoch) {
  const unsigned int d = atomicAdd(&hdr->done, 1u);
  if (d == n_tiles - 1) rearm(hdr, epoch);
}

// The part of the caller's buffer after the header that holds published words (16-byte units, in
// at most two pieces so that the backward's parameter-gradient partials, which its reduction
// launch reads next, stay out of it).
struct ClearSpan {
  uint4* a;
  size_t na;
  uint4* b;
  size_t nb;
};
constexpr uint32_t kEpochMask = 0x3fffffffu;  // bits of the epoch that published words carry

// A forward tile block's end, called by every thread of the block (blocks that refused an
// out-of-range ticket included): counts the block toward the launch's end, and the launch's last
// block re-arms the counter for the next launch (next epoch). Published words carry 30 bits of the
// epoch, so a word written 2^30 launches earlier would carry the tag of the current one. In the
// launch whose next epoch's 30 bits wrap to 0 (the same epoch, so the same branch, for every
// block), the last block therefore zero-fills the whole span first, with the 64 lanes of its wave
// 0 (16 bytes per lane and store): every word any earlier launch left in the buffer (at any
// shape's layout) goes, before any launch of the new cycle reads it. There every block counts
// only after a barrier (all its waves are past their last access to published words) and with
// release-acquire ordering, so the clear lands after every store of the launch and no wave still
// reads what it clears. Every other launch counts with one thread and no barrier. (Code here is in
// the kernel's tail; written this way it leaves the generated code of the kernel's body as it is
// without it.)
__device__ __forceinline__ void finish_launch(LookbackHeader* hdr, uint32_t n_tiles, uint32_t epoch,
                                              const ClearSpan& clr) {
  const bool wrap = ((epoch + 1u) & kEpochMask) == 0u;
  if (!wrap) {
    if (threadIdx.x == 0) finish_block(hdr, n_tiles, epoch);
    return;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    unsigned int d = 0u;
    if (threadIdx.x == 0)
      d = __hip_atomic_fetch_add(&hdr->done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    d = __shfl(d, 0);
    if (d == n_tiles - 1) {
      const uint4 z = make_uint4(0u, 0u, 0u, 0u);
      for (size_t i = threadIdx.x; i < clr.na; i += 64) clr.a[i] = z;
      for (size_t i = threadIdx.x; i < clr.nb; i += 64) clr.b[i] = z;
      if (threadIdx.x == 0) rearm(hdr, epoch);
    }
  }
}
// Tiles at chain positions 1 .. kDirectChunks skip the status scan and wait on their
// predecessors' words directly: the summaries of positions ord-1 .. 1 and the inclusive state of
// position 0, which is what the scan finds for the first round's tiles anyway (at B=8, T=2,048
// the first round holds chunks 0-7 of every chain). One memory round trip fewer for those tiles.
// Cold B=8, T=2,048, three interleaved runs per build: fp32 read 39.5-39.7 -> 38.2-38.5 us,
// bf16 read 32.1 -> 30.7-31.1 us; with 16 positions 38.6-38.9 / 31.2-31.4 us (second-round tiles
// then fetch summaries the scan would not need). FL_DIRECT_CHUNKS is a build switch for
// comparisons (0: never).
#ifndef FL_DIRECT_CHUNKS
#define FL_DIRECT_CHUNKS 8
#endif
constexpr int kDirectChunks = FL_DIRECT_CHUNKS;

constexpr int kLookbackBatch = 2;  // predecessor summaries in flight per wave
// Look-back window: the predecessors whose summaries one round stages in LDS (3 x CT floats
// each): 8W/K, at most 64 (one status load)
constexpr int lookback_window(int K, int W) { return 8 * W / K < 64 ? 8 * W / K : 64; }
// data planes of a tile: P, Br, Bi (summary), Sr, Si (inclusive state)
constexpr int kPlanes = 5;

__device__ __forceinline__ void put_word(uint64_t* p, float v, uint32_t tag) {
  const uint64_t w = ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t word_tag(uint64_t w) { return (uint32_t)(w >> 32); }
__device__ __forceinline__ float word_value(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Wait until every word w[i] (loaded from p[i*stride]) carries `tag`; false if the wait gave up.
template <int N>
__device__ __forceinline__ bool settle_words(uint64_t* p, int stride, uint32_t tag, uint64_t* w,
                                             uint32_t& spins, uint32_t limit) {
  while (true) {
    bool ready = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ready = ready && word_tag(w[i]) == tag;
    if (ready) return true;
    if (++spins > limit) return false;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (word_tag(w[i]) != tag) w[i] = get_word(p + (int64_t)i * stride);
  }
}

// Decoupled look-back of one tile, run by all W waves of the block, with a carry that does not
// depend on timing. The carry is the nearest published inclusive state (INCL) of predecessor
// j0-n (j0 = ord-1) with the summaries (AGG) of predecessors j0-n+1 .. j0 applied to it one by
// one, farthest first, by apply_map with A = lamT * P: exactly how each of those predecessors
// forms its own inclusive state from its carry. Whichever predecessor's inclusive state is found,
// the carry is therefore the same float values (the predecessor j0's inclusive state, bit for
// bit). The n summaries are fetched by all W waves in parallel into s_pred (LDS, kWin x 3 x CT
// floats, nearest first) and applied by wave 0. A tile whose kWin nearest predecessors hold no
// inclusive state, or one whose nearest non-summary predecessor has published nothing yet, waits
// and scans again (an inclusive state reaches every tile within kWin of the lowest unfinished
// one, whose own predecessor is finished). On return wave 0 holds the carry-in in (cr, ci)
// (NaN if a wait gave up after ``limit`` polls, with the error bit set). ``ord`` is the tile's
// position in its chain's processing order; every predecessor is a full tile. Some tiles skip the
// scan and wait on a predecessor set fixed in advance: with span > 0 (a block-order launch whose
// resident blocks hold span positions of every chain per round) the summaries of their round's
// earlier positions and the inclusive state of the previous round's last position; with span 0,
// tiles at positions up to kDirectChunks, from the inclusive state of position 0. The carry is the
// same bits either way (a predecessor's inclusive state with every later summary applied), and the
// wait ends like any other (every predecessor has a lower ticket, so its words are published by a
// block that is resident or done, or the bounded wait gives up).
template <int K, int W, int kWin>
__device__ __forceinline__ void lookback_carry(int ord, int span, int chain, int n_chunks, const uint32_t* st_chain,
                                               uint64_t* data, uint32_t tag_agg, uint32_t tag_incl,
                                               const float* lTr, const float* lTi, bool ok, int lane,
                                               int wave, LookbackHeader* hdr, uint32_t limit,
                                               float* s_pred, float (&s_carry)[2][64 * K],
                                               int (&s_meta)[4], float* cr, float* ci) {
  constexpr int CT = 64 * K;
  static_assert(kWin >= 1 && kWin <= 64, "look-back window of one status load");
  uint32_t spins = 0;
  bool failed = false;
  const int j0 = ord - 1;
  // Status scan (wave 0): statuses of predecessors j0, j0-1, ..., j0-kWin+1 in one load; s_meta
  // gets (n, ready): ready when j0 .. j0-n+1 have published summaries and j0-n its inclusive state.
  auto scan_status = [&]() {
    const int p = j0 - lane;
    const bool in_win = lane < kWin && p >= 0;
    uint32_t s = 0;
    if (in_win) s = __hip_atomic_load(st_chain + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long not_agg = __ballot(!(in_win && s == tag_agg));
    int n = 0, ready = 0;
    if (not_agg != 0ull) {
      const int i0 = __ffsll((long long)not_agg) - 1;
      const uint32_t s_at = __shfl(s, i0);
      n = i0;
      ready = (i0 < kWin && j0 - i0 >= 0 && s_at == tag_incl) ? 1 : 0;
    }
    if (lane == 0) { s_meta[0] = n; s_meta[1] = ready; }
  };
  if (wave == 0) {
    // Direct wait: n summaries and the inclusive state of predecessor j0 - n, without a scan
    int nd = -1;
    if (span > 0) {
      // `span` positions of each chain per round of resident blocks (block order): the tile waits
      // on its own round's earlier summaries and the inclusive state of the previous round's last
      // position (position 0's in the first round)
      const int r0 = (ord / span) * span;
      nd = r0 == 0 ? ord - 1 : ord - r0;
      if (nd >= kWin) nd = -1;
    } else if (ord <= kDirectChunks && ord <= kWin) {
      nd = j0;  // one of the first chunks: the summaries of ord-1 .. 1, position 0's inclusive state
    }
    if (nd >= 0) {
      if (lane == 0) { s_meta[0] = nd; s_meta[1] = 1; }
    } else {
      scan_status();
    }
    if (lane == 0) { s_meta[2] = 0; s_meta[3] = 0; }
  }
  // Each round: barrier, (ready) every wave stages its share of the n summaries and the last wave
  // the inclusive state, barrier, wave 0 applies them or scans the statuses again.
  while (true) {
    __syncthreads();
    if (s_meta[3]) break;
    const int n = s_meta[0], ready = s_meta[1];
    if (ready) {
      const int m = (n + W - 1) / W;
      const int lo = min(wave * m, n), hi = min(lo + m, n);
      // sub-batches of kLookbackBatch predecessors, nearest first (no barrier in between)
      for (int q0 = lo; ok && q0 < hi && !failed; q0 += kLookbackBatch) {
        uint64_t w[kLookbackBatch][3][K];
#pragma unroll
        for (int q = 0; q < kLookbackBatch; ++q) {
          if (q0 + q < hi) {
            uint64_t* dp = data + ((size_t)chain * n_chunks + (j0 - q0 - q)) * kPlanes * CT + lane * K;
#pragma unroll
            for (int k = 0; k < K; ++k) {
              w[q][0][k] = get_word(dp + k);
              w[q][1][k] = get_word(dp + CT + k);
              w[q][2][k] = get_word(dp + 2 * CT + k);
            }
          }
        }
#pragma unroll
        for (int q = 0; q < kLookbackBatch; ++q) {
          if (q0 + q < hi && !failed) {
            uint64_t* dp = data + ((size_t)chain * n_chunks + (j0 - q0 - q)) * kPlanes * CT + lane * K;
            float* sp = s_pred + (size_t)(q0 + q) * 3 * CT + lane * K;
#pragma unroll
            for (int k = 0; k < K; ++k) {
              uint64_t ww[3] = {w[q][0][k], w[q][1][k], w[q][2][k]};
              if (!settle_words<3>(dp + k, CT, tag_agg, ww, spins, limit)) { failed = true; break; }
              sp[k] = word_value(ww[0]);
              sp[CT + k] = word_value(ww[1]);
              sp[2 * CT + k] = word_value(ww[2]);
            }
          }
        }
      }
      if (wave == W - 1 && ok) {  // inclusive state of predecessor j0 - n
        uint64_t* dp = data + ((size_t)chain * n_chunks + (j0 - n)) * kPlanes * CT + lane * K;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          uint64_t ww[2] = {get_word(dp + 3 * CT + k), get_word(dp + 4 * CT + k)};
          if (!settle_words<2>(dp + 3 * CT + k, CT, tag_incl, ww, spins, limit)) { failed = true; break; }
          s_carry[0][lane * K + k] = word_value(ww[0]);
          s_carry[1][lane * K + k] = word_value(ww[1]);
        }
      }
    }
    if (__ballot(failed) != 0ull && lane == 0) {
      report_error(hdr, 1u);
      s_meta[2] = 1;
    }
    __syncthreads();
    if (wave == 0) {
      int done = 0;
      if (s_meta[2]) {
        done = 1;  // a wait gave up: the carry is poisoned
#pragma unroll
        for (int k = 0; k < K; ++k) { cr[k] = poison(); ci[k] = poison(); }
      } else if (ready) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int x = lane * K + k;
          float sr = s_carry[0][x], si = s_carry[1][x];
          for (int i = n - 1; i >= 0; --i) {
            const float* sp = s_pred + (size_t)i * 3 * CT + x;
            apply_map(lTr[k], lTi[k], sp[0], sp[CT], sp[2 * CT], sr, si);
          }
          cr[k] = sr;
          ci[k] = si;
        }
        done = 1;
      } else {
        if (++spins > limit) {
          done = 1;
          if (lane == 0) report_error(hdr, 1u);
#pragma unroll
          for (int k = 0; k < K; ++k) { cr[k] = poison(); ci[k] = poison(); }
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (!done) scan_status();
      if (lane == 0) s_meta[3] = done;
    }
  }
}

// RMSNorm scale of H rows of a wave: lane l returns rsqrt(total / 4C + eps) of row l mod H,
// the total being the sum of the partial words of the n_ctiles channel tiles of the token
// (sg + s * stride: tile s's word of lane l's row), added in the same order by every tile of the
// token (lanes l, l + H, ... take every (64/H)-th tile in turn, then combine by xor shuffles).
// Rows at or past n_valid take no words. A row whose total misses a partial (a wait that gave
// up) gets a NaN scale and the header's error bit.
template <int H>
__device__ __forceinline__ float row_scale(const uint64_t* sg, size_t stride, int n_ctiles,
                                           bool row_valid, uint32_t tag, uint32_t limit,
                                           float inv_n, float eps, LookbackHeader* hdr, int lane) {
  float tot = 0.f;
  bool failed = false;
  if (row_valid) {
    uint32_t spins = 0;
    constexpr int kStride = 64 / H, kBatch = 4;  // lanes per row; words in flight per lane
    for (int s0 = lane / H; s0 < n_ctiles && !failed; s0 += kBatch * kStride) {
      uint64_t w[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int sq = s0 + q * kStride;
        w[q] = sq < n_ctiles ? get_word(const_cast<uint64_t*>(sg) + (size_t)sq * stride) : 0ull;
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int sq = s0 + q * kStride;
        if (sq < n_ctiles && !failed) {
          if (!settle_words<1>(const_cast<uint64_t*>(sg) + (size_t)sq * stride, 0, tag, &w[q],
                               spins, limit)) {
            failed = true;
          } else {
            tot += word_value(w[q]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = H; m < 64; m <<= 1) tot += __shfl_xor(tot, m);
  // the lanes holding a row's words (l, l + H, ...) combine their failures as their sums
  int row_failed = failed ? 1 : 0;
#pragma unroll
  for (int m = H; m < 64; m <<= 1) row_failed |= __shfl_xor(row_failed, m);
  if (__ballot(failed) != 0ull && lane == 0) report_error(hdr, 1u);
  return row_failed ? poison() : rsqrtf(fmaf(tot, inv_n, eps));
}

// Block-order tile of block i with the channel tiles of a row group on one XCD. The dispatcher
// sends block i to XCD i mod 8, so consecutive tickets (the channel tiles of one row group, the
// same rows of raw and read) would land on eight XCDs. Within each window of 8 row groups
// (8 * n_ctiles blocks) the blocks of one XCD instead take the channel tiles of one row group:
// block w*win + 8*j + x takes ticket w*win + x*n_ctiles + j. Every ticket of a window still comes
// from a block of that window, so the block-order progress argument holds (a window's blocks
// are dispatched once the earlier windows' blocks are done, and a window of at most 256 blocks
// fits the chip); a last partial window keeps identity order. Cold B=8, T=2,048: fp32 read
// 39.2 -> 38.6 us, bf16 read 34.6 -> 33.3 us. (With the RMSNorm epilogue it is slower, 36.4 ->
// 39.8 us, and not used there.)
__device__ __forceinline__ uint32_t xcd_grouped_ticket(uint32_t i, uint32_t n_ctiles, uint32_t n_tiles) {
  const uint32_t win = 8u * n_ctiles;
  if (win > 256u) return i;
  const uint32_t w = i / win, u = i - w * win;
  if ((w + 1u) * win > n_tiles) return i;
  return w * win + (u & 7u) * n_ctiles + (u >> 3);
}

// NORM: out = RMSNorm(read) (canon:300-309 applied to canon:1176-1193's read), norm_w [4C],
// sib = per-row partials [n_tiles][W*L] words; otherwise out = read and those are unused.
// LDSIO (bf16 raw, fp32 read, K = 1, every channel tile full, 16-byte aligned raw rows): each
// wave stages its own raw rows in LDS with 16-byte buffer loads that write LDS directly and
// forms the gates from there, and stores read through a per-wave LDS transpose with 16-byte
// stores (the staging region is free again once the look-back's barriers are behind).
template <typename RawT, typename OutT, int K, int L, int W, int OCC, bool NORM, bool LDSIO = false>
__global__ __launch_bounds__(W * 64, OCC) void fl_scan_lookback_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    int n_ctiles, const float* __restrict__ tr, const float* __restrict__ ti,
    const float* __restrict__ gamma, const float* __restrict__ state_in,
    float* __restrict__ state_out, OutT* __restrict__ read, LookbackHeader* hdr,
    uint32_t* status, uint64_t* data, uint32_t n_tiles, int round_span, uint32_t raise_from,
    const float* __restrict__ norm_w, float eps, float inv_n, uint64_t* sib, ClearSpan wrap_clear) {
  // round_span > 0: block order (block i takes tile i), round_span chain positions per round of
  // resident blocks; 0: tickets from the counter. Blocks from raise_from on (the launch's last
  // half-round) issue at raised wave priority.
  const bool in_order = round_span > 0;
  if (blockIdx.x >= raise_from) __builtin_amdgcn_s_setprio(2);
  constexpr int CT = 64 * K;
  constexpr int TC = W * L;
  static_assert(OCC * 4 >= W, "occupancy target below one block per CU");
  // LDSIO stages the look-back's summaries in the raw region (3 x TC x CT bf16)
  constexpr int kWin = LDSIO && TC / 2 < lookback_window(K, W) ? TC / 2 : lookback_window(K, W);
  __shared__ float s_sum[W][3][CT];   // wave summaries (P, Br, Bi)
  __shared__ float s_carry[2][CT];
  __shared__ int s_meta[4];           // look-back: n, ready, failed, done
  __shared__ uint32_t s_tk[2];
  // LDSIO: raw [3][TC][CT] bf16, later the per-wave store staging (W x 4 planes x 4 rows x CT fp32)
  static_assert(!LDSIO || (K == 1 && L % 8 == 0 && sizeof(RawT) == 2),
                "LDS-staged I/O: bf16 raw, one channel per lane, rows in eights");
  constexpr int kStage = 4 * WaveTile<RawT, K, L>::kStageRows * CT;  // floats of a wave's store stage
  static_assert(!LDSIO || W * kStage * 4 <= 3 * TC * CT * 2, "store staging exceeds the raw region");
  static_assert(!LDSIO || kWin * 3 * CT * 4 <= 3 * TC * CT * 2, "look-back staging exceeds the raw region");
  __shared__ __align__(16) bf16_bits s_io[LDSIO ? 3 * TC * CT : 8];
  // look-back staging of predecessor summaries (LDSIO: the raw region, free after the summary
  // barrier until the stores)
  __shared__ float s_pred_own[LDSIO ? 1 : kWin * 3 * CT];
  float* const s_pred = LDSIO ? reinterpret_cast<float*>(s_io) : s_pred_own;

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  uint32_t ticket;
  uint64_t epoch_word = 0;
  if (in_order) {
    // block i takes tile i; the epoch (the counter's high word) is loaded now and stored to LDS
    // once the raw loads issued after it have landed
    ticket = blockIdx.x;
    if constexpr (!NORM) ticket = xcd_grouped_ticket(ticket, (uint32_t)n_ctiles, n_tiles);
    if (wave == 0)
      epoch_word = __hip_atomic_load(&hdr->ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (threadIdx.x == 0) {
      const unsigned long long tk = atomicAdd(&hdr->ticket, 1ull);
      s_tk[0] = (uint32_t)tk;
      s_tk[1] = (uint32_t)(tk >> 32);
    }
    __syncthreads();
    // wave-uniform (SGPR) values: every descriptor and offset built from them stays scalar
    ticket = (uint32_t)uniform((int)s_tk[0]);
    if (ticket >= n_tiles) {  // counter out of range (not re-armed): refuse, terminate
      if (threadIdx.x == 0) report_error(hdr, 2u);
      // counts toward the launch's end like any block (and clears at the epoch wrap if last)
      finish_launch(hdr, n_tiles, (uint32_t)uniform((int)s_tk[1]), wrap_clear);
      return;
    }
  }
  const uint32_t limit = spin_limit_of(hdr);
  const uint32_t n_chains = n_tiles / (uint32_t)n_chunks;
  const int chunk = (int)(ticket / n_chains);
  const int chain = (int)(ticket - (uint32_t)chunk * n_chains);
  const int b = chain / n_ctiles;
  const int ctile = chain - b * n_ctiles;
  const int c0 = ctile * CT + lane * K;
  const bool ok = c0 < C;
  const int t_begin = chunk * TC;
  const bool last_chunk = chunk == n_chunks - 1;

  float lr[K], li[K], gm[K];
  load_params<K>(tr, ti, gamma, c0, ok, lr, li, gm);
  const TileIo io = tile_io<RawT, OutT>(raw, sb, st, read, T, C, b, t_begin, TC, c0);
  WaveTile<RawT, K, L> tile;
  if constexpr (LDSIO) {
    // this wave's rows: 8 rows of one plane per instruction (lane = 8 * row + 16-byte piece)
    const int vo = ctile * CT * (int)sizeof(RawT) + (lane >> 3) * io.raw_row + (lane & 7) * 16;
    constexpr int kRawPolicy = sizeof(OutT) == 2 ? kStreamLoad : 0;  // nt for bf16 output
#pragma unroll
    for (int q = 0; q < 3 * (L / 8); ++q) {
      const int plane = q / (L / 8), r0 = wave * L + (q % (L / 8)) * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          io.raw, (__attribute__((address_space(3))) void*)&s_io[(plane * TC + r0) * CT], 16, vo,
          r0 * io.raw_row + plane * io.raw_plane, 0, kRawPolicy);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the wave reads only the rows it staged itself
    tile.load_lds(&s_io[wave * L * CT], TC * CT, lane, gm);
  } else {
    tile.load(io.raw, io.vo_raw, wave * L * io.raw_row, io.raw_row, io.raw_plane, gm);
  }
  if (in_order && threadIdx.x == 0) s_tk[1] = (uint32_t)(epoch_word >> 32);
  const int n_valid = min(max(T - (t_begin + wave * L), 0), L);
  {
    // full tiles are the only ones whose summary is consumed
    float P[K], Br[K], Bi[K];
    tile.summary(lr, li, P, Br, Bi);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s_sum[wave][0][lane * K + k] = P[k];
      s_sum[wave][1][lane * K + k] = Br[k];
      s_sum[wave][2][lane * K + k] = Bi[k];
    }
  }
  float lLr[K], lLi[K], lTr[K], lTi[K];  // lam^L, lam^TC
#pragma unroll
  for (int k = 0; k < K; ++k) {
    cpow(lr[k], li[k], L, lLr[k], lLi[k]);
    cpow(lLr[k], lLi[k], W, lTr[k], lTi[k]);
  }
  __syncthreads();
  const uint32_t epoch = (uint32_t)uniform((int)s_tk[1]);
  const uint32_t tag_agg = ((epoch & 0x3fffffffu) << 2) | kTagAgg;
  const uint32_t tag_incl = ((epoch & 0x3fffffffu) << 2) | kTagIncl;

  const uint32_t tile_id = (uint32_t)chain * (uint32_t)n_chunks + (uint32_t)chunk;
  uint32_t* st_chain = status + (size_t)chain * n_chunks;
  uint64_t* dt = data + (size_t)tile_id * kPlanes * CT + lane * K;
  float TP[K], TBr[K], TBi[K];  // tile summary (wave 0)
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) { TP[k] = 1.f; TBr[k] = 0.f; TBi[k] = 0.f; }
    for (int u = 0; u < W; ++u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        apply_map(lLr[k], lLi[k], s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], TBr[k], TBi[k]);
        TP[k] *= s_sum[u][0][x];
      }
    }
    if (chunk > 0 && !last_chunk) {
      if (ok) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          put_word(dt + 0 * CT + k, TP[k], tag_agg);
          put_word(dt + 1 * CT + k, TBr[k], tag_agg);
          put_word(dt + 2 * CT + k, TBi[k], tag_agg);
        }
      }
      if (lane == 0)
        __hip_atomic_store(st_chain + chunk, tag_agg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // carry-in of the tile (wave 0's registers)
  float cr[K], ci[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    cr[k] = (ok && state_in) ? state_in[(int64_t)b * 2 * C + c0 + k] : 0.f;
    ci[k] = (ok && state_in) ? state_in[(int64_t)b * 2 * C + C + c0 + k] : 0.f;
  }
  if (chunk > 0)
    // span 0: the first-positions rule only. Direct waits in later rounds too (the previous
    // round's last inclusive state, which is often late here) measured slower for the forward:
    // cold B=8, T=2,048 fp32 read 38.2-38.4 -> 38.9-39.1 us, RMSNorm epilogue 34.7-34.9 ->
    // 35.1-36.0 us
    lookback_carry<K, W, kWin>(chunk, 0, chain, n_chunks, st_chain, data, tag_agg, tag_incl, lTr, lTi,
                               ok, lane, wave, hdr, limit, s_pred, s_carry, s_meta, cr, ci);
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s_carry[0][lane * K + k] = cr[k];
      s_carry[1][lane * K + k] = ci[k];
    }
    // publish the inclusive state (every tile but the last of its chain has a successor)
    if (!last_chunk) {
      if (ok) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          float sr = cr[k], si = ci[k];
          apply_map(lTr[k], lTi[k], TP[k], TBr[k], TBi[k], sr, si);
          put_word(dt + 3 * CT + k, sr, tag_incl);
          put_word(dt + 4 * CT + k, si, tag_incl);
        }
      }
      if (lane == 0)
        __hip_atomic_store(st_chain + chunk, tag_incl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();

  if (NORM ? n_valid > 0 : (ok && n_valid > 0)) {
    float sr[K], si[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      sr[k] = s_carry[0][lane * K + k];
      si[k] = s_carry[1][lane * K + k];
    }
    for (int u = 0; u < wave; ++u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        apply_map(lLr[k], lLi[k], s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], sr[k], si[k]);
      }
    }
    if constexpr (NORM) {
      // The tile's read values are kept for the stores; the partial sums of squares of its rows
      // are published for the sibling tiles of the token. (Rows
      // exchanged in two or four parts, each published as soon as formed so that one part's
      // exchange overlaps the next part's pass: cold B=8, T=2,048 35.8 -> 36.5 / 38.9 us.)
      float v[L][4], ss[L];
      // (LDSIO: every channel of the tile lies below C, so every lane is in range)
      tile.template norm_values<L>(0, n_valid, LDSIO || ok, lr[0], li[0], sr[0], si[0], v, ss);
      const int row = lane & (L - 1);
      const uint32_t tag_sib = ((epoch & 0x3fffffffu) << 2) | kTagSib;
      static_assert(L == 16 && kWin * 3 * CT >= W * 1024, "row sums staged in the look-back region");
      // the look-back's staging region is free again (its last barrier is behind): 1024 floats
      // per wave
      const float part = wave_row_sums_lds(ss, lane, s_pred + wave * 1024);
      const int prow = lane >> 2;  // the row whose sum this lane holds
      if ((lane & 3) == 0 && prow < n_valid) put_word(sib + (size_t)ticket * TC + wave * L + prow, part, tag_sib);
      // the norm weights are needed only after the exchange: load them now, under its wait
      float nw[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) nw[p] = ok ? norm_w[p * C + c0] : 0.f;
      // sibling s's word of this lane's row
      const uint64_t* const sg = sib + ((size_t)chunk * n_chains + (size_t)b * n_ctiles) * TC + wave * L + row;
      const float scale = row_scale<L>(sg, TC, n_ctiles, row < n_valid, tag_sib, limit, inv_n, eps,
                                       hdr, lane);
      if constexpr (LDSIO) {
        float* stage = reinterpret_cast<float*>(s_io) + wave * kStage;
        WaveTile<RawT, K, L>::template store_norm_lds<OutT, L>(
            io.read, lane, 0, wave * L * io.read_row, io.read_row, io.read_plane,
            ctile * CT * (int)sizeof(OutT), stage, v, scale, nw);
      } else {
        WaveTile<RawT, K, L>::template store_norm<OutT, L>(io.read, io.vo_read, 0,
                                                           wave * L * io.read_row, io.read_row,
                                                           io.read_plane, n_valid, ok, v, scale, nw);
      }
    } else if constexpr (LDSIO) {
      float* stage = reinterpret_cast<float*>(s_io) + wave * kStage;
      if (n_valid == L)  // every row in range: the row checks fold away
        tile.template materialize_lds<OutT>(io.read, lane, wave * L * io.read_row, io.read_row,
                                            io.read_plane, ctile * CT * (int)sizeof(OutT), L,
                                            stage, lr, li, sr, si);
      else
        tile.template materialize_lds<OutT>(io.read, lane, wave * L * io.read_row, io.read_row,
                                            io.read_plane, ctile * CT * (int)sizeof(OutT), n_valid,
                                            stage, lr, li, sr, si);
    } else {
      tile.template materialize<OutT>(io.read, io.vo_read, wave * L * io.read_row, io.read_row,
                                     io.read_plane, n_valid, lr, li, sr, si);
    }
    if (ok && state_out != nullptr && t_begin + wave * L + n_valid == T) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        state_out[(int64_t)b * 2 * C + c0 + k] = sr[k];
        state_out[(int64_t)b * 2 * C + C + c0 + k] = si[k];
      }
    }
  }

  // the last block of the launch re-arms the counter for the next launch (next epoch)
  finish_launch(hdr, n_tiles, epoch, wrap_clear);
}

// ------------------------------------------------------------------------------------------
// Backward scan (fl_scan_backward): the adjoint of the forward recurrence (canon:625-910,
// 1020-1105), one scan launch with tiles taken in reverse time order, then the parameter-gradient
// reduction launch.
//
// With U_t = dL/ds_t and D_t = dL/d disp_t (grad_read), the gradient reaching s_t from later
// steps, c_t, obeys (a_t = (1 - v_t) lam, conj = complex conjugate)
//   G_t = U_t + c_t,    c_{t-1} = conj(a_t) G_t + conj(v_t lam) D_t
//                              = conj(lam) [(1 - v_t)(c_t + U_t) + v_t D_t],    c_{T-1} = grad_state_out,
// a diagonal affine recurrence like the forward one: n steps map c to conj(lam)^n prod(1-v) c + Q.
// Tiles summarise, publish and look back as in the forward pass, with processing position
// ord = n_chunks - 1 - chunk; the only partial tile (the end of the sequence) is ord 0, which
// never publishes a summary. Per step, with p = s_{t-1} (the forward read, state_in at t = 0):
//   dzr = gamma v Re(G) (1 - tanh^2 zr),  dzi = gamma v Im(G) (1 - tanh^2 zi),
//   dv  = Re(conj(D) lam p) - Re(conj(G) lam p) + gamma Re(conj(G) inj),  dzv = dv v (1 - v/0.9),
//   dlam += (1 - v) G conj(p) + v D conj(p),   dgamma += v Re(conj(G) inj),
// and c_{-1} = grad_state_in. Parameter gradients are summed per tile (each lane over its steps,
// then the waves in order) into per-tile partials, which a second launch
// (fl_param_grad_reduce_kernel) adds up over the tiles of each channel tile in a fixed order
// (deterministic).
// The second pass needs s_{t-1} at every step, which the reference reads back from the forward's
// read (canon:841-850); here each wave recomputes it with the forward recurrence from the state
// entering its first row (the read at the row before, state_in or 0 at the sequence start),
// which takes 8 of the 36 bytes per channel and step off the backward's traffic.
// PF (K = 1, every channel tile full, 16-byte aligned raw rows): the second pass's z_r, z_i are
// staged in LDS by 16-byte buffer loads that write LDS directly, issued with the first pass's
// loads, so that no load latency follows the look-back.
// ------------------------------------------------------------------------------------------
template <typename RawT, typename GradT, int K, int L, int W, int OCC, bool PF = false>
__global__ __launch_bounds__(W * 64, OCC) void fl_scan_backward_kernel(
    const RawT* __restrict__ raw, int64_t sb, int64_t st, int T, int C, int n_chunks,
    int n_ctiles, const float* __restrict__ tr, const float* __restrict__ ti,
    const float* __restrict__ gamma, const float* __restrict__ state_in,
    const float* __restrict__ read, const float* __restrict__ grad_read,
    const float* __restrict__ grad_state_out, GradT* __restrict__ grad_raw,
    float* __restrict__ grad_state_in, LookbackHeader* hdr, uint32_t* status, uint64_t* data,
    float* __restrict__ part, uint32_t n_tiles, uint32_t n_chains, int round_span) {
  const bool in_order = round_span > 0;  // as in the forward kernel
  constexpr int CT = 64 * K;
  constexpr int TC = W * L;
  static_assert(OCC * 4 >= W, "occupancy target below one block per CU");
  __shared__ float s_sum[W][3][CT];   // wave maps (P, Qr, Qi)
  __shared__ float s_part[W][3][CT];  // parameter-gradient partials (dlam re, im, dgamma)
  __shared__ float s_carry[2][CT];
  __shared__ int s_meta[4];
  __shared__ uint32_t s_tk[2];
  // look-back staging of predecessor summaries (a narrower window keeps fp32 raw staging at two
  // blocks per CU)
  constexpr int kWin = (PF && sizeof(RawT) == 4) ? lookback_window(K, W) / 2 : lookback_window(K, W);
  __shared__ float s_pred[kWin * 3 * CT];
  // PF: z_r, z_i [TC][CT] (RawT)
  constexpr int kPfRaw = TC * CT * (int)sizeof(RawT);
  static_assert(!PF || (K == 1 && L % 8 == 0), "LDS staging: one channel per lane, rows in eights");
  __shared__ __align__(16) unsigned char s_pf[PF ? 2 * kPfRaw : 16];

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  uint32_t ticket;
  uint64_t epoch_word = 0;
  if (in_order) {  // block i takes tile i, as in the forward kernel
    ticket = blockIdx.x;
    if (wave == 0)
      epoch_word = __hip_atomic_load(&hdr->ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (threadIdx.x == 0) {
      const unsigned long long tk = atomicAdd(&hdr->ticket, 1ull);
      s_tk[0] = (uint32_t)tk;
      s_tk[1] = (uint32_t)(tk >> 32);
    }
    __syncthreads();
    // wave-uniform (SGPR) values: every descriptor and offset built from them stays scalar
    ticket = (uint32_t)uniform((int)s_tk[0]);
    if (ticket >= n_tiles) {  // counter out of range (not re-armed): refuse, terminate
      if (threadIdx.x == 0) {
        report_error(hdr, 2u);
        finish_block(hdr, n_tiles, s_tk[1]);
      }
      return;
    }
  }
  const uint32_t limit = spin_limit_of(hdr);
  const int ord = (int)(ticket / n_chains);
  const int chain = (int)(ticket - (uint32_t)ord * n_chains);
  const int chunk = n_chunks - 1 - ord;
  const int b = chain / n_ctiles;
  const int ctile = chain - b * n_ctiles;
  const int c0 = ctile * CT + lane * K;
  const bool ok = c0 < C;
  const int t_begin = chunk * TC;
  const bool last_ord = ord == n_chunks - 1;

  float lr[K], li[K], gm[K], clr[K], cli[K];
  load_params<K>(tr, ti, gamma, c0, ok, lr, li, gm);
#pragma unroll
  for (int k = 0; k < K; ++k) { clr[k] = lr[k]; cli[k] = -li[k]; }
  const int w0 = t_begin + wave * L;
  const int n_valid = min(max(T - w0, 0), L);

  // buffers over the tile's rows from row t_begin of batch row b: raw (rows of st elements),
  // grad_read (rows of 4C), grad_raw (rows of 3C); rows past T read as 0 and drop their stores
  const int rows = min(T - t_begin, TC);
  const rsrc_t r_raw = make_rsrc(raw + (int64_t)b * sb + (int64_t)t_begin * st,
                                 (uint32_t)(((int64_t)(rows - 1) * st + 3 * (int64_t)C) * sizeof(RawT)));
  const rsrc_t r_grd = make_rsrc(grad_read + ((int64_t)b * T + t_begin) * 4 * C,
                                 (uint32_t)((int64_t)rows * 4 * C * 4));
  const rsrc_t r_out = make_rsrc(grad_raw + ((int64_t)b * T + t_begin) * 3 * C,
                                 (uint32_t)((int64_t)rows * 3 * C * sizeof(GradT)));
  const int vo_raw = c0 * (int)sizeof(RawT), vo_f = c0 * 4, vo_out = c0 * (int)sizeof(GradT);
  const int raw_row = (int)(st * (int64_t)sizeof(RawT)), raw_plane = C * (int)sizeof(RawT);
  const int grd_row = 4 * C * 4, f_plane = C * 4;
  const int out_row = 3 * C * (int)sizeof(GradT), out_plane = C * (int)sizeof(GradT);

  // this wave's rows: U, D (grad_read) and v (from z_v), kept for both passes
  float uR[L][K], uI[L][K], dR[L][K], dI[L][K], gv[L][K];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const int so = (wave * L + j) * grd_row;
    RawLoad<float, K, kStreamLoad>::run(r_grd, vo_f, so, uR[j]);
    RawLoad<float, K, kStreamLoad>::run(r_grd, vo_f, so + f_plane, uI[j]);
    RawLoad<float, K, kStreamLoad>::run(r_grd, vo_f, so + 2 * f_plane, dR[j]);
    RawLoad<float, K, kStreamLoad>::run(r_grd, vo_f, so + 3 * f_plane, dI[j]);
    float zv[K];
    RawLoad<RawT, K>::run(r_raw, vo_raw, (wave * L + j) * raw_row + 2 * raw_plane, zv);
#pragma unroll
    for (int k = 0; k < K; ++k)
      gv[j][k] = kVacancyMax * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zv[k] * -kLog2e));
  }
  // the state entering the wave's first row (loaded now, used after the look-back)
  float s0r[K], s0i[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s0r[k] = 0.f;
    s0i[k] = 0.f;
    if (ok && n_valid > 0 && w0 > 0) {
      const float* rp = read + ((int64_t)b * T + w0 - 1) * 4 * C + c0 + k;
      s0r[k] = rp[0];
      s0i[k] = rp[C];
    } else if (ok && w0 == 0 && state_in) {
      s0r[k] = state_in[(int64_t)b * 2 * C + c0 + k];
      s0i[k] = state_in[(int64_t)b * 2 * C + C + c0 + k];
    }
  }
  // Only a wave with valid rows stages them: it waits for its loads before its second pass
  // reads them. A wave past T issues none, since one still in flight when the block retires
  // would write into LDS that a later block on the CU then owns.
  if (PF && n_valid > 0) {
    // raw planes: a row of CT channels is kRawLanes 16-byte pieces, kRawRows rows per load
    constexpr int kRawLanes = CT * (int)sizeof(RawT) / 16, kRawRows = 64 / kRawLanes;
    const int vo_r = ctile * CT * (int)sizeof(RawT) + (lane / kRawLanes) * raw_row + (lane % kRawLanes) * 16;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int i = 0; i < L / kRawRows; ++i) {
        const int r0 = wave * L + i * kRawRows;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r_raw, (__attribute__((address_space(3))) void*)&s_pf[p * kPfRaw + r0 * CT * (int)sizeof(RawT)],
            16, vo_r, r0 * raw_row + p * raw_plane, 0, 0);
      }
  }
  if (in_order && threadIdx.x == 0) s_tk[1] = (uint32_t)(epoch_word >> 32);
  {
    // wave map from its right edge to its left edge over its valid rows (reverse order)
    float P[K], Qr[K], Qi[K];
#pragma unroll
    for (int k = 0; k < K; ++k) { P[k] = 1.f; Qr[k] = 0.f; Qi[k] = 0.f; }
#pragma unroll
    for (int j = L - 1; j >= 0; --j) {
      if (j < n_valid) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const float keep = 1.f - gv[j][k];
          const float xr = fmaf(keep, Qr[k] + uR[j][k], gv[j][k] * dR[j][k]);
          const float xi = fmaf(keep, Qi[k] + uI[j][k], gv[j][k] * dI[j][k]);
          cmul(clr[k], cli[k], xr, xi, Qr[k], Qi[k]);
          P[k] *= keep;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s_sum[wave][0][lane * K + k] = P[k];
      s_sum[wave][1][lane * K + k] = Qr[k];
      s_sum[wave][2][lane * K + k] = Qi[k];
    }
  }
  float cLr[K], cLi[K], cTr[K], cTi[K];  // conj(lam)^L, conj(lam)^TC
#pragma unroll
  for (int k = 0; k < K; ++k) {
    cpow(clr[k], cli[k], L, cLr[k], cLi[k]);
    cpow(cLr[k], cLi[k], W, cTr[k], cTi[k]);
  }
  // conj(lam)^(valid rows of wave u): L except in the (partial) last tile of the sequence
  auto wave_pow = [&](int u, int k, float& pr, float& pi) {
    const int nu = min(max(T - (t_begin + u * L), 0), L);
    if (nu == L) { pr = cLr[k]; pi = cLi[k]; } else { cpow(clr[k], cli[k], nu, pr, pi); }
  };
  __syncthreads();
  const uint32_t epoch = (uint32_t)uniform((int)s_tk[1]);
  const uint32_t tag_agg = ((epoch & 0x3fffffffu) << 2) | kTagAgg;
  const uint32_t tag_incl = ((epoch & 0x3fffffffu) << 2) | kTagIncl;

  const uint32_t tile_id = (uint32_t)chain * (uint32_t)n_chunks + (uint32_t)ord;
  uint32_t* st_chain = status + (size_t)chain * n_chunks;
  uint64_t* dt = data + (size_t)tile_id * kPlanes * CT + lane * K;
  // map of a full tile (ord > 0; wave 0): published as its summary, and applied to its carry for
  // its inclusive state the way the look-back of later tiles applies it
  float TP[K], TBr[K], TBi[K];
#pragma unroll
  for (int k = 0; k < K; ++k) { TP[k] = 1.f; TBr[k] = 0.f; TBi[k] = 0.f; }
  if (wave == 0 && ord > 0) {
    for (int u = W - 1; u >= 0; --u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        apply_map(cLr[k], cLi[k], s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], TBr[k], TBi[k]);
        TP[k] *= s_sum[u][0][x];
      }
    }
  }
  if (wave == 0 && ord > 0 && !last_ord) {  // full tile with a successor: publish its map
    if (ok) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        put_word(dt + 0 * CT + k, TP[k], tag_agg);
        put_word(dt + 1 * CT + k, TBr[k], tag_agg);
        put_word(dt + 2 * CT + k, TBi[k], tag_agg);
      }
    }
    if (lane == 0)
      __hip_atomic_store(st_chain + ord, tag_agg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  float cr[K], ci[K];  // carry entering the tile's last row
#pragma unroll
  for (int k = 0; k < K; ++k) {
    cr[k] = (ok && grad_state_out) ? grad_state_out[(int64_t)b * 2 * C + c0 + k] : 0.f;
    ci[k] = (ok && grad_state_out) ? grad_state_out[(int64_t)b * 2 * C + C + c0 + k] : 0.f;
  }
  if (ord > 0)
    // direct waits in every round of a block-order launch: cold B=8, T=2,048 (four rounds of
    // 64-step tiles) 59.8-60.3 -> 58.4-59.0 us against the first-positions rule alone
    lookback_carry<K, W, kWin>(ord, round_span, chain, n_chunks, st_chain, data, tag_agg, tag_incl,
                               cTr, cTi, ok, lane, wave, hdr, limit, s_pred, s_carry, s_meta, cr, ci);
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s_carry[0][lane * K + k] = cr[k];
      s_carry[1][lane * K + k] = ci[k];
    }
    if (!last_ord) {  // the carry leaving the tile's first row, for the tile before it in time
      if (ok) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          float sr = cr[k], si = ci[k];
          if (ord > 0) {
            apply_map(cTr[k], cTi[k], TP[k], TBr[k], TBi[k], sr, si);
          } else {  // the end of the sequence (maybe partial): its waves' maps one by one
            for (int u = W - 1; u >= 0; --u) {
              const int x = lane * K + k;
              float pr, pi;
              wave_pow(u, k, pr, pi);
              apply_map(pr, pi, s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], sr, si);
            }
          }
          put_word(dt + 3 * CT + k, sr, tag_incl);
          put_word(dt + 4 * CT + k, si, tag_incl);
        }
      }
      if (lane == 0)
        __hip_atomic_store(st_chain + ord, tag_incl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();

  float gtr[K], gti[K], ggm[K];
#pragma unroll
  for (int k = 0; k < K; ++k) { gtr[k] = 0.f; gti[k] = 0.f; ggm[k] = 0.f; }
  if (n_valid > 0) {
    float car[K], cai[K];  // carry entering this wave's last valid row
#pragma unroll
    for (int k = 0; k < K; ++k) {
      car[k] = s_carry[0][lane * K + k];
      cai[k] = s_carry[1][lane * K + k];
    }
    for (int u = W - 1; u > wave; --u) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        float pr, pi;
        wave_pow(u, k, pr, pi);
        apply_map(pr, pi, s_sum[u][0][x], s_sum[u][1][x], s_sum[u][2][x], car[k], cai[k]);
      }
    }
    // z_r, z_i of the wave's rows (staged in LDS, or every load issued before the dependent
    // chain; rows past T read as 0 through the descriptor bound), then the forward recurrence
    // from the state entering the first row: p = s_{t-1} of every row, and z -> tanh(z) in place
    float zr[L][K], zi[L][K], pr[L][K], pi[L][K];
    if constexpr (PF) {
      __builtin_amdgcn_s_waitcnt(0);  // the wave reads only the rows it staged itself
      const RawT* szr = reinterpret_cast<const RawT*>(s_pf);
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int x = (wave * L + j) * CT + lane;
        zr[j][0] = raw_value(szr[x]);
        zi[j][0] = raw_value(szr[TC * CT + x]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < L; ++j) {
        RawLoad<RawT, K>::run(r_raw, vo_raw, (wave * L + j) * raw_row, zr[j]);
        RawLoad<RawT, K>::run(r_raw, vo_raw, (wave * L + j) * raw_row + raw_plane, zi[j]);
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float sr = s0r[k], si = s0i[k];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        // tanh = 1 - 2 / (1 + e^{2z}), as in the forward gates
        zr[j][k] = fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zr[j][k] * (2.0f * kLog2e))), 1.0f);
        zi[j][k] = fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(zi[j][k] * (2.0f * kLog2e))), 1.0f);
        pr[j][k] = sr;
        pi[j][k] = si;
        if (j + 1 < n_valid) {  // s_j, needed as p by row j + 1
          const float v = gv[j][k], gvv = gm[k] * v;
          float mr, mi;
          cmul(lr[k], li[k], sr, si, mr, mi);
          sr = fmaf(1.f - v, mr, gvv * zr[j][k]);
          si = fmaf(1.f - v, mi, gvv * zi[j][k]);
        }
      }
    }
#pragma unroll
    for (int j = L - 1; j >= 0; --j) {
      if (j < n_valid) {
        float ozr[K], ozi[K], ozv[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const float v = gv[j][k], keep = 1.f - v;
          const float injr = zr[j][k], inji = zi[j][k];
          // every product and sum written as explicit fmas (see cmul)
          const float Gr = uR[j][k] + car[k], Gi = uI[j][k] + cai[k];
          const float p_r = pr[j][k], p_i = pi[j][k];
          float mr, mi;  // lam p
          cmul(lr[k], li[k], p_r, p_i, mr, mi);
          const float cb = fmaf(injr, Gr, inji * Gi);      // Re(conj(G) inj)
          const float dDm = fmaf(dR[j][k], mr, dI[j][k] * mi), dGm = fmaf(Gr, mr, Gi * mi);
          const float dv = fmaf(gm[k], cb, dDm - dGm);
          const float gp_r = fmaf(Gr, p_r, Gi * p_i), gp_i = fmaf(Gi, p_r, -(Gr * p_i));
          const float dp_r = fmaf(dR[j][k], p_r, dI[j][k] * p_i), dp_i = fmaf(dI[j][k], p_r, -(dR[j][k] * p_i));
          gtr[k] = fmaf(keep, gp_r, fmaf(v, dp_r, gtr[k]));
          gti[k] = fmaf(keep, gp_i, fmaf(v, dp_i, gti[k]));
          ggm[k] = fmaf(v, cb, ggm[k]);
          const float gvv = gm[k] * v;
          ozr[k] = (gvv * Gr) * fmaf(-injr, injr, 1.0f);
          ozi[k] = (gvv * Gi) * fmaf(-inji, inji, 1.0f);
          ozv[k] = (dv * v) * fmaf(-v, 1.0f / kVacancyMax, 1.0f);
          const float xr = fmaf(keep, Gr, v * dR[j][k]);
          const float xi = fmaf(keep, Gi, v * dI[j][k]);
          cmul(clr[k], cli[k], xr, xi, car[k], cai[k]);
        }
        if (ok) {  // lanes past C would land in the next plane of the row
          const int so = (wave * L + j) * out_row;
          ReadStore<GradT, K>::run(r_out, vo_out, so, ozr);
          ReadStore<GradT, K>::run(r_out, vo_out, so + out_plane, ozi);
          ReadStore<GradT, K>::run(r_out, vo_out, so + 2 * out_plane, ozv);
        }
      }
    }
    if (w0 == 0 && grad_state_in != nullptr && ok) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        grad_state_in[(int64_t)b * 2 * C + c0 + k] = car[k];
        grad_state_in[(int64_t)b * 2 * C + C + c0 + k] = cai[k];
      }
    }
  }
  // parameter-gradient partials of the tile: waves summed in order
#pragma unroll
  for (int k = 0; k < K; ++k) {
    s_part[wave][0][lane * K + k] = gtr[k];
    s_part[wave][1][lane * K + k] = gti[k];
    s_part[wave][2][lane * K + k] = ggm[k];
  }
  __syncthreads();
  // The tiles of a channel tile, in ticket order, are its rows r = ord * B + b: the tile writes its
  // row of partials (part[ctile][plane][r][CT]), which fl_param_grad_reduce_kernel adds up after
  // this launch.
  {
    const int n_b = (int)(n_chains / (uint32_t)n_ctiles);
    const int n_rows = n_chunks * n_b;
    const int row = ord * n_b + b;
    if (wave == 0 && ok) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int x = lane * K + k;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f;
        for (int u = 0; u < W; ++u) { a0 += s_part[u][0][x]; a1 += s_part[u][1][x]; a2 += s_part[u][2][x]; }
        float* pr = part + ((size_t)ctile * 3 * n_rows + row) * CT + x;
        pr[0] = a0;
        pr[(size_t)n_rows * CT] = a1;
        pr[(size_t)2 * n_rows * CT] = a2;
      }
    }
  }

  // the last block of the launch re-arms the counter for the next launch (next epoch); the
  // reduction launch clears the workspace when that epoch wraps the published words' tags
  if (threadIdx.x == 0) finish_block(hdr, n_tiles, epoch);
}

// Parameter gradients (dlam = grad_tr + i grad_ti and dgamma, summed over batch rows and steps):
// the backward's per-tile partials part[ctile][plane][row][64] (plane 0: Re dlam, 1: Im dlam,
// 2: dgamma) added up over the n_rows rows of each channel tile. One block per (channel tile,
// plane), lane = channel: wave w adds its run of rows in order, then wave 0 adds the 16 wave sums
// in order, so the sums do not depend on timing.
// It also keeps the backward workspace's published words valid across the epoch's wrap: it runs
// after the scan launch has ended, and when the epoch that launch armed for the next one has the
// low 30 bits 0 (the tags of a new cycle), its blocks zero-fill `wrap_clear` (the workspace after
// the header, less the partials) between them, so that no word left 2^30 launches earlier can
// pass for one of the new cycle. The scan launch itself then needs no code for it.
__global__ __launch_bounds__(1024) void fl_param_grad_reduce_kernel(const float* __restrict__ part,
                                                                   int n_rows, int C,
                                                                   float* __restrict__ grad_tr,
                                                                   float* __restrict__ grad_ti,
                                                                   float* __restrict__ grad_gamma,
                                                                   const LookbackHeader* hdr,
                                                                   ClearSpan wrap_clear) {
  constexpr int CT = 64, NW = 16, kBatch = 32;
  __shared__ float s_acc[NW][CT];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int ctile = (int)blockIdx.x / 3, plane = (int)blockIdx.x - 3 * ctile;
  // the header words first, so that their round trip overlaps the partials' (the scan launch
  // that set them has ended)
  const uint32_t err = __hip_atomic_load(const_cast<unsigned int*>(&hdr->error), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t next_epoch = (uint32_t)(__hip_atomic_load(&hdr->ticket, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT) >> 32);
  const float* base = part + ((size_t)ctile * 3 + plane) * n_rows * CT + lane;
  const int rpw = (n_rows + NW - 1) / NW;
  const int r0 = min(wave * rpw, n_rows), r1 = min(r0 + rpw, n_rows);
  float acc = 0.f;
  for (int r = r0; r < r1; r += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) v[q] = r + q < r1 ? base[(size_t)(r + q) * CT] : 0.f;
#pragma unroll
    for (int q = 0; q < kBatch; ++q)
      if (r + q < r1) acc += v[q];
  }
  s_acc[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float t = 0.f;
    for (int u = 0; u < NW; ++u) t += s_acc[u][lane];
    // a tile whose block refused an out-of-range ticket (error bit 1, set by the scan launch)
    // wrote no partials: its rows hold an earlier call's values, so the sums are poisoned
    if (err & 2u) t = poison();
    const int c = ctile * CT + lane;
    if (c < C) (plane == 0 ? grad_tr : plane == 1 ? grad_ti : grad_gamma)[c] = t;
  }
  if ((next_epoch & kEpochMask) == 0u) {  // uniform over the grid
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < wrap_clear.na; i += stride)
      wrap_clear.a[i] = z;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < wrap_clear.nb; i += stride)
      wrap_clear.b[i] = z;
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
    float keep, br, bi;
    gates(zr[k], zi[k], zv[k], kVacancyMax * gm[k], keep, br, bi);
    float mr, mi;
    cmul(lr[k], li[k], sr[k], si[k], mr, mi);
    dr[k] = fmaf(-keep, mr, mr);
    di[k] = fmaf(-keep, mi, mi);
    sr[k] = fmaf(keep, mr, br);
    si[k] = fmaf(keep, mi, bi);
  }
  Store<K>::run(s, sr);
  Store<K>::run(s + C, si);
  float* o = read_t + (int64_t)b * 4 * C + c0;
  Store<K>::run(o, sr);
  Store<K>::run(o + C, si);
  Store<K>::run(o + 2 * C, dr);
  Store<K>::run(o + 3 * C, di);
}

// Decode step with the RMSNorm epilogue: one block per batch row. Pass 1 forms the row's sum of
// squares of the four read values over all C channels; pass 2 updates the state in place and
// stores (value * rsqrt(mean + eps)) * weight. With NPER > 0 (C <= 256 * NPER) each thread
// keeps its NPER channels' values in registers between the passes; with NPER = 0 pass 2
// recomputes them (any C). Each channel is owned by one thread in both passes, so the in-place
// update cannot race.
constexpr int kDecodeNormThreads = 256;

__device__ __forceinline__ void decode_one(float zr, float zi, float zv, float lr, float li,
                                           float gm, float& sr, float& si, float& dr, float& di) {
  float keep, br, bi;
  gates(zr, zi, zv, kVacancyMax * gm, keep, br, bi);
  float mr, mi;
  cmul(lr, li, sr, si, mr, mi);
  dr = fmaf(-keep, mr, mr);
  di = fmaf(-keep, mi, mi);
  sr = fmaf(keep, mr, br);
  si = fmaf(keep, mi, bi);
}

__device__ __forceinline__ void store_out(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_out(bf16_bits* p, float v) { *p = (bf16_bits)bf16_bits_of(v); }

template <typename RawT, typename OutT, int NPER>
__global__ __launch_bounds__(kDecodeNormThreads) void fl_decode_norm_kernel(
    const RawT* __restrict__ raw_t, int64_t sb, int C, const float* __restrict__ tr,
    const float* __restrict__ ti, const float* __restrict__ gamma, float* __restrict__ state,
    const float* __restrict__ norm_w, float eps, float inv_n, OutT* __restrict__ out_t) {
  __shared__ float s_red[kDecodeNormThreads / 64];
  const int b = blockIdx.x;
  const RawT* p = raw_t + (int64_t)b * sb;
  float* s = state + (int64_t)b * 2 * C;
  OutT* o = out_t + (int64_t)b * 4 * C;
  float acc = 0.f;
  if constexpr (NPER > 0) {
    float vr[NPER], vi[NPER], vdr[NPER], vdi[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int c = threadIdx.x + i * kDecodeNormThreads;
      vr[i] = vi[i] = vdr[i] = vdi[i] = 0.f;
      if (c < C) {
        float z[3];
        vr[i] = s[c];
        vi[i] = s[C + c];
        Load<RawT, 1>::run(p + c, &z[0]);
        Load<RawT, 1>::run(p + C + c, &z[1]);
        Load<RawT, 1>::run(p + 2 * C + c, &z[2]);
        decode_one(z[0], z[1], z[2], tr[c], ti[c], gamma[c], vr[i], vi[i], vdr[i], vdi[i]);
        acc = fmaf(vr[i], vr[i], acc);
        acc = fmaf(vi[i], vi[i], acc);
        acc = fmaf(vdr[i], vdr[i], acc);
        acc = fmaf(vdi[i], vdi[i], acc);
      }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) acc += __shfl_xor(acc, m);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeNormThreads / 64; ++w) tot += s_red[w];
    const float scale = rsqrtf(fmaf(tot, inv_n, eps));
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int c = threadIdx.x + i * kDecodeNormThreads;
      if (c < C) {
        s[c] = vr[i];
        s[C + c] = vi[i];
        store_out(o + c, (vr[i] * scale) * norm_w[c]);
        store_out(o + C + c, (vi[i] * scale) * norm_w[C + c]);
        store_out(o + 2 * C + c, (vdr[i] * scale) * norm_w[2 * C + c]);
        store_out(o + 3 * C + c, (vdi[i] * scale) * norm_w[3 * C + c]);
      }
    }
    return;
  }
  for (int c = threadIdx.x; c < C; c += kDecodeNormThreads) {
    float z[3], sr = s[c], si = s[C + c], dr, di;
    Load<RawT, 1>::run(p + c, &z[0]);
    Load<RawT, 1>::run(p + C + c, &z[1]);
    Load<RawT, 1>::run(p + 2 * C + c, &z[2]);
    decode_one(z[0], z[1], z[2], tr[c], ti[c], gamma[c], sr, si, dr, di);
    acc = fmaf(sr, sr, acc);
    acc = fmaf(si, si, acc);
    acc = fmaf(dr, dr, acc);
    acc = fmaf(di, di, acc);
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) acc += __shfl_xor(acc, m);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kDecodeNormThreads / 64; ++w) tot += s_red[w];
  const float scale = rsqrtf(fmaf(tot, inv_n, eps));
  for (int c = threadIdx.x; c < C; c += kDecodeNormThreads) {
    float z[3], sr = s[c], si = s[C + c], dr, di;
    Load<RawT, 1>::run(p + c, &z[0]);
    Load<RawT, 1>::run(p + C + c, &z[1]);
    Load<RawT, 1>::run(p + 2 * C + c, &z[2]);
    decode_one(z[0], z[1], z[2], tr[c], ti[c], gamma[c], sr, si, dr, di);
    s[c] = sr;
    s[C + c] = si;
    store_out(o + c, (sr * scale) * norm_w[c]);
    store_out(o + C + c, (si * scale) * norm_w[C + c]);
    store_out(o + 2 * C + c, (dr * scale) * norm_w[2 * C + c]);
    store_out(o + 3 * C + c, (di * scale) * norm_w[3 * C + c]);
  }
}

// ------------------------------------------------------------------------------------------
// Boundary scan of the softpatch (BoundaryStateMixer, v3:441-464 / v6:318-338):
//   s[b,t,r] = a[b,t] * s[b,t-1,r] + drive[b,t,r],   s[b,-1,:] = state_in or 0,
// the real-valued first-order recurrence that the reference runs through
// hierarchical_scan(a, drive, block=32) with a = (1 - boundary) broadcast over the rank.
// Block = (batch row, 64 channels), W waves; wave w owns steps [w*S, (w+1)*S). Pass 1 forms
// each wave's map (prod a, state from 0) over its steps, the waves' carries are composed in LDS,
// pass 2 re-runs from the carry and stores. Lane <-> channel, so each step is one coalesced
// 256-byte load and store; a[b,t] is the same for the whole wave.
// ------------------------------------------------------------------------------------------
constexpr int kBoundaryWaves = 16;

__global__ __launch_bounds__(kBoundaryWaves * 64) void fl_boundary_scan_kernel(
    const float* __restrict__ a, const float* __restrict__ drive, int T, int R,
    const float* __restrict__ state_in, float* __restrict__ state_out, float* __restrict__ out) {
  __shared__ float s_p[kBoundaryWaves][64], s_s[kBoundaryWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int b = blockIdx.x;
  const int r = blockIdx.y * 64 + lane;
  const bool ok = r < R;
  const int span = (T + kBoundaryWaves - 1) / kBoundaryWaves;
  const int t0 = min(wave * span, T), t1 = min(t0 + span, T);
  const float* ab = a + (int64_t)b * T;
  const float* db = drive + (int64_t)b * T * R + r;
  float* ob = out + (int64_t)b * T * R + r;
  float p = 1.f, sv = 0.f;
  for (int t = t0; t < t1; ++t) {
    const float at = ab[t];
    const float d = ok ? db[(int64_t)t * R] : 0.f;
    sv = fmaf(at, sv, d);
    p *= at;
  }
  s_p[wave][lane] = p;
  s_s[wave][lane] = sv;
  __syncthreads();
  float c = (ok && state_in) ? state_in[(int64_t)b * R + r] : 0.f;
  for (int u = 0; u < wave; ++u) c = fmaf(s_p[u][lane], c, s_s[u][lane]);
  for (int t = t0; t < t1; ++t) {
    const float at = ab[t];
    const float d = ok ? db[(int64_t)t * R] : 0.f;
    c = fmaf(at, c, d);
    if (ok) ob[(int64_t)t * R] = c;
  }
  if (ok && state_out && wave == kBoundaryWaves - 1) {
    // the last wave ends at T (or holds the composed carry when its span is empty)
    state_out[(int64_t)b * R + r] = c;
  }
}

// ------------------------------------------------------------------------------------------
// Field block elementwise tail (canon:1193-1195, 1219-1221, RMSNorm 300-309, SwiGLU 312-325),
// fused for the inference path. Each value is rounded exactly where the stock ops round it:
// an op on bf16 tensors computes in fp32 and rounds its result to bf16.
//   fl_gate_residual_norm:  gate = sigmoid(g), prod = out * gate (in the GEMM output dtype G),
//                           x1 = x + prod (in the residual dtype X), h = RMSNorm(x1) * w (fp32
//                           math, rounded to X) — one block per row, x1 kept in registers.
//   fl_swiglu:              out = silu(gate) * up with [gate | up] = the packed GEMM output.
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float round_as(float v);
template <>
__device__ __forceinline__ float round_as<float>(float v) { return v; }
template <>
__device__ __forceinline__ float round_as<bf16_bits>(float v) { return __uint_as_float(bf16_bits_of(v) << 16); }

template <typename T>
__device__ __forceinline__ float load_as(const T* p);
template <>
__device__ __forceinline__ float load_as<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_as<bf16_bits>(const bf16_bits* p) { return __uint_as_float((uint32_t)*p << 16); }

constexpr int kTailThreads = 256;

template <typename XT, typename GT, int NPER>
__global__ __launch_bounds__(kTailThreads) void fl_gate_residual_norm_kernel(
    const XT* __restrict__ x, const GT* __restrict__ out, const GT* __restrict__ gpre,
    int64_t gstride, int dim, const float* __restrict__ w, float eps, float inv_dim,
    XT* __restrict__ x_new, XT* __restrict__ normed) {
  __shared__ float s_red[kTailThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * dim;
  const GT* grow = gpre + (int64_t)blockIdx.x * gstride;
  auto residual = [&](int c) {
    const float gate = round_as<GT>(1.0f / (1.0f + expf(-load_as<GT>(grow + c))));
    const float prod = round_as<GT>(load_as<GT>(out + base + c) * gate);
    return round_as<XT>(load_as<XT>(x + base + c) + prod);
  };
  float v[NPER > 0 ? NPER : 1];
  float acc = 0.f;
  if constexpr (NPER > 0) {
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int c = threadIdx.x + i * kTailThreads;
      v[i] = c < dim ? residual(c) : 0.f;
      acc = fmaf(v[i], v[i], acc);
    }
  } else {
    for (int c = threadIdx.x; c < dim; c += kTailThreads) {
      const float r = residual(c);
      acc = fmaf(r, r, acc);
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) acc += __shfl_xor(acc, m);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = acc;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kTailThreads / 64; ++i) tot += s_red[i];
  const float scale = rsqrtf(fmaf(tot, inv_dim, eps));
  if constexpr (NPER > 0) {
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int c = threadIdx.x + i * kTailThreads;
      if (c < dim) {
        store_out(x_new + base + c, v[i]);
        store_out(normed + base + c, (v[i] * scale) * w[c]);
      }
    }
  } else {
    for (int c = threadIdx.x; c < dim; c += kTailThreads) {
      const float r = residual(c);
      store_out(x_new + base + c, r);
      store_out(normed + base + c, (r * scale) * w[c]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void fl_swiglu_kernel(const T* __restrict__ gu, int64_t rows,
                                                        int hidden, T* __restrict__ out) {
  const int64_t n = rows * hidden;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / hidden;
    const int j = (int)(i - r * hidden);
    const float g = load_as<T>(gu + r * 2 * hidden + j);
    const float u = load_as<T>(gu + r * 2 * hidden + hidden + j);
    const float sg = round_as<T>(g / (1.0f + expf(-g)));
    store_out(out + i, sg * u);
  }
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

// Look-back tilings: (K channels per lane, L steps per wave, W waves per block, OCC target
// waves per SIMD, which caps the VGPR budget so that OCC*4/W blocks share a CU).
// Variant 0 is the default; the others are selectable for tuning (algo >> 8). Every one reaches
// its occupancy target without scratch (a 32-step tiling at 4 waves per SIMD spilled, the
// default at 6 stayed at 4, and two channels per lane with 16-step waves spilled 2 VGPRs at 3).
struct LookbackTiling {
  int k, l, w, occ;
};
constexpr LookbackTiling kLookbackTilings[] = {
    {1, 16, 8, 4}, {1, 16, 8, 2}, {1, 32, 4, 3}, {2, 16, 4, 2}, {2, 8, 8, 4}, {1, 16, 4, 4},
};
constexpr int kNumLookbackTilings = sizeof(kLookbackTilings) / sizeof(kLookbackTilings[0]);
// The default tiling with LDS-staged raw loads and read stores (LDSIO) is what variant 0 runs for
// the inputs it takes (bf16 raw, fp32 read, C a multiple of 64, 16-byte aligned rows); variant
// kLdsIoVariant asks for it explicitly and kRegIoVariant for the default tiling with register
// loads and stores on every input.
constexpr int kLdsIoVariant = kNumLookbackTilings;
constexpr int kRegIoVariant = kNumLookbackTilings + 1;
// The RMSNorm epilogue runs with the default tiling only; a group of channel tiles must be
// resident together, so its size n_ctiles = C/64 is capped (C <= 4096).
constexpr LookbackTiling kNormTiling = kLookbackTilings[0];
constexpr int64_t kNormMaxCtiles = 64;

// Workspace layout, fixed for a shape whatever the algorithm or tiling:
//   [header 2 KiB][status: max tiles x u32][data: max tiles x 5 x CT x u64]
//   [sib: tiles x TC x u64 of the RMSNorm tiling][chunked3 floats]
// Status words and data words are only ever written as tagged words (by any tiling), and the
// three-phase buffers have their own region, so a word left by another call can never carry
// the current launch's tag.
struct WorkspaceLayout {
  size_t status_off, data_off, sib_off, chunked3_off, bytes;
};

struct LookbackGeom {
  int n_chunks, n_ctiles;
  uint32_t n_tiles;
};

LookbackGeom lookback_geom(int64_t B, int64_t T, int64_t C, int CT, int TC) {
  LookbackGeom g;
  g.n_chunks = (int)cdiv(T, TC);
  g.n_ctiles = (int)cdiv(C, CT);
  g.n_tiles = (uint32_t)(B * g.n_ctiles * (int64_t)g.n_chunks);
  return g;
}

WorkspaceLayout workspace_layout(int64_t B, int64_t T, int64_t C) {
  size_t max_tiles = 0, max_data = 0;
  for (int v = 0; v < kNumLookbackTilings; ++v) {
    const LookbackTiling tl = kLookbackTilings[v];
    for (int k = tl.k; k >= 1; k /= 2) {  // narrowed variants have smaller CT
      const LookbackGeom g = lookback_geom(B, T, C, 64 * k, tl.l * tl.w);
      const size_t data = (size_t)g.n_tiles * kPlanes * (64 * k) * sizeof(uint64_t);
      if (g.n_tiles > max_tiles) max_tiles = g.n_tiles;
      if (data > max_data) max_data = data;
    }
  }
  WorkspaceLayout w;
  w.status_off = kHeaderBytes;
  w.data_off = w.status_off + (size_t)cdiv((int64_t)max_tiles * 4, 256) * 256;
  w.sib_off = w.data_off + (size_t)cdiv((int64_t)max_data, 256) * 256;
  {
    const LookbackTiling tl = kNormTiling;
    const LookbackGeom g = lookback_geom(B, T, C, 64 * tl.k, tl.l * tl.w);
    w.chunked3_off = w.sib_off + (size_t)cdiv((int64_t)g.n_tiles * tl.l * tl.w * 8, 256) * 256;
  }
  w.bytes = w.chunked3_off + (size_t)(B * cdiv(T, kChunkT) * C) * 5 * sizeof(float);
  return w;
}

template <typename RawT, typename OutT, int K>
int launch_chunked3(const RawT* raw, int64_t B, int64_t T, int64_t C, int64_t sb, int64_t st,
                    const float* tr, const float* ti, const float* gamma, const float* state_in,
                    float* state_out, OutT* read, float* agg, float* carry, hipStream_t stream) {
  constexpr int CT = 64 * K;
  const int n_chunks = (int)cdiv(T, kChunkT);
  const dim3 grid((unsigned)n_chunks, (unsigned)cdiv(C, CT), (unsigned)B);
  fl_chunk_summary_kernel<RawT, K, 8, 8><<<grid, 8 * 64, 0, stream>>>(
      raw, sb, st, (int)T, (int)C, n_chunks, tr, ti, gamma, agg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_status(e);
  const dim3 cgrid((unsigned)cdiv(C, 64), (unsigned)B);
  fl_chunk_carry_kernel<<<cgrid, kCarryWaves * 64, 0, stream>>>(agg, (int)C, n_chunks, tr, ti,
                                                                 state_in, carry);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_status(e);
  fl_chunk_materialize_kernel<RawT, OutT, K, 8, 8><<<grid, 8 * 64, 0, stream>>>(
      raw, sb, st, (int)T, (int)C, n_chunks, tr, ti, gamma, carry, read, state_out);
  return hip_status(hipGetLastError());
}

template <typename RawT, typename OutT>
int dispatch_chunked3(int k, const void* raw, int64_t B, int64_t T, int64_t C, int64_t sb,
                      int64_t st, const float* tr, const float* ti, const float* gamma,
                      const float* state_in, float* state_out, void* read, float* agg,
                      float* carry, hipStream_t stream) {
  const RawT* r = static_cast<const RawT*>(raw);
  OutT* o = static_cast<OutT*>(read);
  switch (k) {
    case 4:
      return launch_chunked3<RawT, OutT, 4>(r, B, T, C, sb, st, tr, ti, gamma, state_in,
                                            state_out, o, agg, carry, stream);
    case 2:
      return launch_chunked3<RawT, OutT, 2>(r, B, T, C, sb, st, tr, ti, gamma, state_in,
                                            state_out, o, agg, carry, stream);
    default:
      return launch_chunked3<RawT, OutT, 1>(r, B, T, C, sb, st, tr, ti, gamma, state_in,
                                            state_out, o, agg, carry, stream);
  }
}

struct NormArgs {
  const float* weight;  // [4C], nullptr: no epilogue
  float eps;
};

// Where a launch keeps its look-back state: the header, the status words, the tagged data words
// and (RMSNorm epilogue) the per-row partials; and the span cleared when the epoch wraps.
struct WsRegions {
  LookbackHeader* hdr;
  uint32_t* status;
  uint64_t* data;
  uint64_t* sib;
  ClearSpan clr;
};

// The whole buffer after the header (`bytes` as the caller gave it), in 16-byte units.
ClearSpan clear_span_after_header(void* buffer, size_t bytes) {
  char* p = static_cast<char*>(buffer) + kHeaderBytes;
  const size_t n = bytes > kHeaderBytes ? (bytes - kHeaderBytes) / 16 : 0;
  return {reinterpret_cast<uint4*>(p), n, nullptr, 0};
}

WsRegions regions_of(void* workspace, size_t workspace_bytes_given, int64_t B, int64_t T, int64_t C) {
  const WorkspaceLayout lay = workspace_layout(B, T, C);
  char* ws = static_cast<char*>(workspace);
  return {reinterpret_cast<LookbackHeader*>(ws), reinterpret_cast<uint32_t*>(ws + lay.status_off),
          reinterpret_cast<uint64_t*>(ws + lay.data_off), reinterpret_cast<uint64_t*>(ws + lay.sib_off),
          clear_span_after_header(workspace, workspace_bytes_given)};
}

constexpr int kMaxDevices = 64;  // devices the library keeps per-device state for

// CU count of the stream's device, read once per device (256 if the query fails).
int device_cus(hipStream_t stream) {
  static std::atomic<int> cus[kMaxDevices];
  int dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = -1;
  int n = dev >= 0 ? cus[dev].load(std::memory_order_relaxed) : 0;
  if (n <= 0) {
    if (dev < 0 || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    if (dev >= 0) cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Chain positions per round of resident blocks in a block-order launch: blocks_per_cu x the
// device's CU count, divided among n_chains chains; at least 1. A hint for the look-back's direct
// waits only: results and progress do not depend on it.
int round_span(hipStream_t stream, int blocks_per_cu, int64_t n_chains) {
  const int64_t span = (int64_t)blocks_per_cu * device_cus(stream) / (n_chains > 0 ? n_chains : 1);
  return span < 1 ? 1 : (int)(span > (1 << 20) ? (1 << 20) : span);
}

// First block of the forward launch's raised tail: the last half-round of resident blocks
// (blocks_per_cu x CUs / 2) when at least a full round of blocks comes before it, else n_tiles
// (none). Those blocks start while the previous round's blocks still hold the other slots of their
// CUs, and on a SIMD the older waves issue first, so they would otherwise finish last and set the
// kernel's end. In the launch's first round of resident blocks the same stagger is what lets the
// second round start early, so the first round is never raised. Issue order only: results do not
// depend on it.
uint32_t tail_raise_from(hipStream_t stream, int blocks_per_cu, uint32_t n_tiles) {
  const int64_t resident = (int64_t)blocks_per_cu * device_cus(stream);
  const int64_t from = (int64_t)n_tiles - resident / 2;
  return from >= resident ? (uint32_t)from : n_tiles;
}

template <typename RawT, typename OutT, int K, int L, int W, int OCC, bool NORM, bool LDSIO = false>
int launch_lookback(const void* raw, int64_t B, int64_t T, int64_t C, int64_t sb, int64_t st,
                    const float* tr, const float* ti, const float* gamma, const float* state_in,
                    float* state_out, void* read, const WsRegions& rg, NormArgs norm,
                    hipStream_t stream) {
  constexpr int CT = 64 * K;
  const LookbackGeom g = lookback_geom(B, T, C, CT, W * L);
  // Ticket order. Short chains (<= 64 chunks): block i takes tile i, no ticket atomic on the
  // critical path (B=8, T=2,048 with the RMSNorm epilogue 41.4 -> 37.0 us: the channel tiles of a
  // token start together, one per XCD). This relies on the dispatcher issuing each XCD's share of
  // the grid in block order: then the lowest unfinished tile (or RMSNorm sibling group) is always
  // resident, since every block resident ahead of it on its XCD has a lower index. Long chains:
  // tickets from one counter, whose serialisation hands them out in the order blocks actually
  // start, which the look-back needs to keep up (B=1, T=65,536: 155 us; 203 us in block order,
  // 216 us with eight counters).
  const bool in_order = g.n_chunks <= 64;
  const int span = in_order ? round_span(stream, OCC * 4 / W, (int64_t)g.n_tiles / g.n_chunks) : 0;
  // raised tail: plain scans only. The RMSNorm epilogue loses with counter tickets (B=1,
  // T=65,536: 142.3 -> 144.0 us, where the plain scan gains 148.9 -> 147.6 us) and gains at most
  // 0.5 us in block order (B=8, T=2,048); it keeps plain priority.
  const uint32_t raise_from = NORM ? g.n_tiles : tail_raise_from(stream, OCC * 4 / W, g.n_tiles);
  fl_scan_lookback_kernel<RawT, OutT, K, L, W, OCC, NORM, LDSIO><<<g.n_tiles, W * 64, 0, stream>>>(
      static_cast<const RawT*>(raw), sb, st, (int)T, (int)C, g.n_chunks, g.n_ctiles, tr, ti,
      gamma, state_in, state_out, static_cast<OutT*>(read), rg.hdr, rg.status, rg.data,
      g.n_tiles, span, raise_from, norm.weight, norm.eps, (float)(1.0 / (4.0 * (double)C)),
      rg.sib, rg.clr);
  return hip_status(hipGetLastError());
}

template <typename RawT, typename OutT>
int dispatch_lookback(int variant, int k, const void* raw, int64_t B, int64_t T, int64_t C,
                      int64_t sb, int64_t st, const float* tr, const float* ti, const float* gamma,
                      const float* state_in, float* state_out, void* read, const WsRegions& ws,
                      NormArgs norm, hipStream_t s) {
#define FL_LB(KK, LL, WW, OO)                                                                  \
  if (kk == KK && tl.l == LL && tl.w == WW && tl.occ == OO)                                     \
    return launch_lookback<RawT, OutT, KK, LL, WW, OO, false>(raw, B, T, C, sb, st, tr, ti,    \
                                                              gamma, state_in, state_out, read, \
                                                              ws, norm, s);
  if (norm.weight != nullptr) {  // RMSNorm epilogue: the default tiling (K = 1, no narrowing)
    constexpr LookbackTiling tl = kNormTiling;
    static_assert(tl.k == 1, "the RMSNorm tiling must not need alignment narrowing");
    return launch_lookback<RawT, OutT, tl.k, tl.l, tl.w, tl.occ, true>(
        raw, B, T, C, sb, st, tr, ti, gamma, state_in, state_out, read, ws, norm, s);
  }
  if constexpr (sizeof(OutT) == 2) {
    // bf16 read: the default tiling only (its K = 1 needs no alignment narrowing)
    const LookbackTiling tl = kLookbackTilings[0];
    const int kk = tl.k;
    FL_LB(1, 16, 8, 4)
  } else {
    const LookbackTiling tl = kLookbackTilings[variant];
    const int kk = tl.k <= k ? tl.k : k;  // never wider than the alignment allows
    FL_LB(1, 16, 8, 4) FL_LB(1, 16, 8, 2) FL_LB(1, 32, 4, 3) FL_LB(2, 16, 4, 2) FL_LB(2, 8, 8, 4)
    FL_LB(1, 16, 4, 4)
    // narrowed K (alignment): same L, W, OCC
    FL_LB(1, 16, 4, 2) FL_LB(1, 8, 8, 4)
  }
#undef FL_LB
  return FL_ERR_INVALID_ARGUMENT;
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

// Shape limits: grid.y = C/(64K) and grid.z = B stay <= 65535; the buffer descriptors of a
// tile (its rows only, at most 128 rows of at most 4 MiB) and every byte offset inside them
// stay below 2^31; the look-back tile count stays below 2^31.
constexpr int64_t kMaxB = 65535;
constexpr int64_t kMaxC = (int64_t)1 << 16;
constexpr int64_t kMaxT = (int64_t)1 << 30;
constexpr int64_t kMaxRowBytes = (int64_t)1 << 22;  // 512 rows of a tile stay below 2^31 bytes

size_t workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (B <= 0 || T <= 0 || C <= 0) return 0;
  return workspace_layout(B, T, C).bytes;
}

// Backward tiling (K channels per lane, L steps per wave, W waves, OCC waves per SIMD) and its
// workspace: [header 2 KiB][status: tiles x u32][data: tiles x 5 x CT x u64]
// [parameter-gradient partials: channel tiles x 3 planes x (n_chunks x B) rows x CT fp32]
constexpr LookbackTiling kBwdTiling = {1, 8, 8, 4};

struct BwdLayout {
  LookbackGeom g;
  int n_rows;  // partial rows per channel tile (tiles of the channel tile: n_chunks x B)
  size_t status_off, data_off, part_off, bytes;
};

BwdLayout bwd_layout(int64_t B, int64_t T, int64_t C) {
  BwdLayout w;
  const int CT = 64 * kBwdTiling.k;
  w.g = lookback_geom(B, T, C, CT, kBwdTiling.l * kBwdTiling.w);
  w.status_off = kHeaderBytes;
  w.data_off = w.status_off + (size_t)cdiv((int64_t)w.g.n_tiles * 4, 256) * 256;
  w.part_off = w.data_off + (size_t)cdiv((int64_t)w.g.n_tiles * kPlanes * CT * 8, 256) * 256;
  w.n_rows = (int)(B * (int64_t)w.g.n_chunks);
  w.bytes = w.part_off + (size_t)cdiv((int64_t)w.g.n_tiles * 3 * CT * 4, 256) * 256;
  return w;
}

template <typename RawT, typename GradT>
int launch_backward(const void* raw, int64_t B, int64_t T, int64_t C, int64_t sb, int64_t st,
                    const float* tr, const float* ti, const float* gamma, const float* state_in,
                    const float* read, const float* grad_read, const float* grad_state_out,
                    void* grad_raw, float* grad_tr, float* grad_ti, float* grad_gamma,
                    float* grad_state_in, void* workspace, size_t workspace_bytes_given,
                    hipStream_t stream) {
  constexpr LookbackTiling tl = kBwdTiling;
  constexpr int CT = 64 * tl.k;
  const BwdLayout lay = bwd_layout(B, T, C);
  const LookbackGeom& g = lay.g;
  char* ws = static_cast<char*>(workspace);
  // cleared by the reduction launch when the epoch wraps: the buffer after the header, except
  // this call's partials, which that launch reads (every tile writes its row of them, which
  // overwrites whatever an earlier launch left there)
  const size_t part_end = lay.part_off + (size_t)cdiv((int64_t)g.n_tiles * 3 * CT * 4, 16) * 16;
  ClearSpan clr{reinterpret_cast<uint4*>(ws + kHeaderBytes), (lay.part_off - kHeaderBytes) / 16,
                reinterpret_cast<uint4*>(ws + part_end),
                workspace_bytes_given > part_end ? (workspace_bytes_given - part_end) / 16 : 0};
  const int64_t n_chains = B * (int64_t)g.n_ctiles;
  // ticket order as in the forward launch: block order for short chains, one counter otherwise
  const bool in_order = g.n_chunks <= 64;
  const int span = in_order ? round_span(stream, tl.occ * 4 / tl.w, n_chains) : 0;
  // LDS-staged second-pass raw: every channel tile full, raw rows 16-byte aligned
  const int64_t esz = (int64_t)sizeof(RawT);
  const bool pf = FL_BWD_PREFETCH && C % CT == 0 && aligned(raw, 16) && (st * esz) % 16 == 0 &&
                  (B == 1 || (sb * esz) % 16 == 0);
#define FL_BWK(PF)                                                                               \
  fl_scan_backward_kernel<RawT, GradT, tl.k, tl.l, tl.w, tl.occ, PF><<<g.n_tiles, tl.w * 64, 0, stream>>>( \
      static_cast<const RawT*>(raw), sb, st, (int)T, (int)C, g.n_chunks, g.n_ctiles, tr, ti, gamma, \
      state_in, read, grad_read, grad_state_out, static_cast<GradT*>(grad_raw), grad_state_in,     \
      reinterpret_cast<LookbackHeader*>(ws),                                                      \
      reinterpret_cast<uint32_t*>(ws + lay.status_off), reinterpret_cast<uint64_t*>(ws + lay.data_off), \
      reinterpret_cast<float*>(ws + lay.part_off), g.n_tiles, (uint32_t)n_chains, span)
  if (pf) {
    FL_BWK(true);
  } else {
    FL_BWK(false);
  }
#undef FL_BWK
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_status(e);
  static_assert(CT == 64, "fl_param_grad_reduce_kernel sums rows of 64 channels");
  fl_param_grad_reduce_kernel<<<(unsigned)(g.n_ctiles * 3), 1024, 0, stream>>>(
      reinterpret_cast<const float*>(ws + lay.part_off), lay.n_rows, (int)C, grad_tr, grad_ti, grad_gamma,
      reinterpret_cast<const LookbackHeader*>(ws), clr);
  return hip_status(hipGetLastError());
}

}  // namespace

extern "C" {

const char* fl_version(void) { return "fields_amd 0.3 gfx950"; }

size_t fl_scan_workspace_bytes(int64_t B, int64_t T, int64_t C) { return workspace_bytes(B, T, C); }

}  // extern "C"

namespace {

int scan_impl(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
              int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
              const float* gamma, const float* state_in, float* state_out, void* read,
              int read_dtype, void* workspace, size_t workspace_bytes_given, int algo,
              NormArgs norm, void* stream, const WsRegions* fixed = nullptr) {
  if (raw_dtype != FL_DTYPE_F32 && raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (read_dtype != FL_DTYPE_F32 && read_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  const int base_algo = algo & 0xff;
  const int variant = algo >> 8;
  if (base_algo != FL_ALGO_AUTO && base_algo != FL_ALGO_CHUNKED3 && base_algo != FL_ALGO_LOOKBACK)
    return FL_ERR_INVALID_ARGUMENT;
  if (variant < 0 || variant > kRegIoVariant) return FL_ERR_INVALID_ARGUMENT;
  if (B <= 0 || T <= 0 || C <= 0 || B > kMaxB || C > kMaxC || T > kMaxT)
    return FL_ERR_INVALID_ARGUMENT;
  if (raw_stride_t < 3 * C || raw_stride_b < 0) return FL_ERR_INVALID_ARGUMENT;
  if (B > 1 && raw_stride_b < (T - 1) * raw_stride_t + 3 * C) return FL_ERR_INVALID_ARGUMENT;
  const int64_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  // within a tile, raw and read rows are addressed through 32-bit buffer offsets
  const int64_t osz = read_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (raw_stride_t * esz > kMaxRowBytes || 4 * C * osz > kMaxRowBytes) return FL_ERR_INVALID_ARGUMENT;
  if (B * cdiv(T, 32) * cdiv(C, 64) >= ((int64_t)1 << 31)) return FL_ERR_INVALID_ARGUMENT;
  if (!raw || !tr || !ti || !gamma || !read) return FL_ERR_INVALID_ARGUMENT;
  if (fixed == nullptr) {
    const size_t need = workspace_bytes(B, T, C);
    if (!workspace || workspace_bytes_given < need) return FL_ERR_WORKSPACE;
    if (!aligned(workspace, 256)) return FL_ERR_INVALID_ARGUMENT;
  } else if (base_algo == FL_ALGO_CHUNKED3 || variant != 0 || norm.weight != nullptr) {
    return FL_ERR_INVALID_ARGUMENT;  // fixed regions: the default look-back launch only
  }
  if (!aligned(raw, esz) || !aligned(read, osz)) return FL_ERR_INVALID_ARGUMENT;
  if ((state_in && !aligned(state_in, 4)) || (state_out && !aligned(state_out, 4)))
    return FL_ERR_INVALID_ARGUMENT;
  if (norm.weight != nullptr) {
    // the epilogue exists on the look-back path only; a group of C/64 channel tiles must be
    // resident together
    if (base_algo == FL_ALGO_CHUNKED3 || variant != 0) return FL_ERR_INVALID_ARGUMENT;
    if (cdiv(C, 64 * kNormTiling.k) > kNormMaxCtiles) return FL_ERR_INVALID_ARGUMENT;
    if (!aligned(norm.weight, 4) || !(norm.eps >= 0.f)) return FL_ERR_INVALID_ARGUMENT;
  }

  int k = pick_k(raw_dtype, raw, C, raw_stride_b, raw_stride_t, read, nullptr, nullptr);
  if (osz == 2) {  // bf16 read: K values are stored as K*2 bytes
    while (k > 1 && !aligned(read, 2 * k)) k /= 2;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool raw16 = raw_dtype == FL_DTYPE_BF16, out16 = read_dtype == FL_DTYPE_BF16;
  const WsRegions rg = fixed != nullptr ? *fixed : regions_of(workspace, workspace_bytes_given, B, T, C);
  if (base_algo == FL_ALGO_CHUNKED3) {
    const int64_t n_chunks = cdiv(T, kChunkT);
    float* agg = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                          workspace_layout(B, T, C).chunked3_off);
    float* carry = agg + B * n_chunks * 3 * C;
#define FL_C3(R, O)                                                                              \
  return dispatch_chunked3<R, O>(k, raw, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma,   \
                                 state_in, state_out, read, agg, carry, s);
    if (raw16 && out16) FL_C3(bf16_bits, bf16_bits)
    if (raw16) FL_C3(bf16_bits, float)
    if (out16) FL_C3(float, bf16_bits)
    FL_C3(float, float)
#undef FL_C3
  }
  // LDS-staged I/O: bf16 raw with 16-byte aligned rows, every 64-channel tile full, read (fp32
  // or bf16, with or without the RMSNorm epilogue) 16-byte aligned
  const bool ldsio_ok = raw16 && C % 64 == 0 && aligned(raw, 16) && raw_stride_t % 8 == 0 &&
                        (B == 1 || raw_stride_b % 8 == 0) && aligned(read, 16);
  if ((variant == 0 || variant == kLdsIoVariant) && ldsio_ok) {
    constexpr LookbackTiling tl = kLookbackTilings[0];
    static_assert(tl.k == kNormTiling.k && tl.l == kNormTiling.l && tl.w == kNormTiling.w,
                  "the RMSNorm epilogue runs with the default tiling");
#define FL_LDSIO(O, N)                                                                          \
  return launch_lookback<bf16_bits, O, tl.k, tl.l, tl.w, tl.occ, N, true>(                      \
      raw, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma, state_in, state_out, read,        \
      rg, norm, s);
    if (norm.weight != nullptr) {
      if (out16) { FL_LDSIO(bf16_bits, true) }
      FL_LDSIO(float, true)
    }
    if (out16) { FL_LDSIO(bf16_bits, false) }
    FL_LDSIO(float, false)
#undef FL_LDSIO
  }
  const int lb_variant = variant >= kLdsIoVariant ? 0 : variant;
#define FL_LBD(R, O)                                                                          \
  return dispatch_lookback<R, O>(lb_variant, k, raw, B, T, C, raw_stride_b, raw_stride_t, tr,  \
                                 ti, gamma, state_in, state_out, read, rg, norm, s);
  if (raw16 && out16) FL_LBD(bf16_bits, bf16_bits)
  if (raw16) FL_LBD(bf16_bits, float)
  if (out16) FL_LBD(float, bf16_bits)
  FL_LBD(float, float)
#undef FL_LBD
}

}  // namespace

// ------------------------------------------------------------------------------------------
// No-allocation variant of fl_scan_forward (fl_scan_forward_static): the look-back state lives in
// a file-scope device array, `scratch`, one copy per GPU for the life of the process, instead of
// a caller-provided workspace. Layout: [header 2 KiB][status: kStaticMaxTiles x u32]
// [data: kStaticMaxTiles x 5 planes x 64 channels x u64]. Launches of the default look-back tiling
// (64-channel x 128-step tiles) use it; every call on a GPU shares that GPU's array, so calls that
// overlap on one GPU race. Nothing in it has to start at zero per call: every word carries the
// epoch that each launch advances. It is zero-filled once, at the first call on each device.
// ------------------------------------------------------------------------------------------
namespace {
constexpr uint32_t kStaticMaxTiles = FL_STATIC_MAX_TILES;
constexpr size_t kStaticStatusOff = kHeaderBytes;
constexpr size_t kStaticDataOff = kStaticStatusOff + ((size_t)kStaticMaxTiles * 4 + 255) / 256 * 256;
constexpr size_t kStaticScratchBytes = kStaticDataOff + (size_t)kStaticMaxTiles * kPlanes * 64 * 8;
static_assert(kStaticScratchBytes == FL_STATIC_SCRATCH_BYTES, "scratch size stated in fields_amd.h");
static_assert(kStaticScratchBytes % 16 == 0, "zero-filled in 16-byte stores");
}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

__global__ __launch_bounds__(256) void fl_fill_zero_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

struct StaticScratch {
  std::mutex m;
  char* ptr[kMaxDevices] = {};  // device address of each GPU's `scratch` (null: not set up)
};

StaticScratch& static_scratch_state() {
  static StaticScratch st;
  return st;
}

// This GPU's copy of `scratch` (the stream's device): at the first call on a device its address
// is looked up with that device current and it is zero-filled on `stream` (so that first call
// must not be under stream capture: a captured fill would re-run on every replay).
int static_scratch(hipStream_t stream, char** out) {
  int dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return hip_status(e);
  if (dev < 0 || dev >= kMaxDevices) return FL_ERR_INVALID_ARGUMENT;
  StaticScratch& st = static_scratch_state();
  std::lock_guard<std::mutex> lock(st.m);
  if (st.ptr[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(stream, &cs)) != hipSuccess) return hip_status(e);
    if (cs != hipStreamCaptureStatusNone) return FL_ERR_CAPTURE;
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_status(e);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_status(e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return hip_status(e);
    if (p == nullptr) return FL_ERR_HIP_BASE + (int)hipErrorInvalidSymbol;
    fl_fill_zero_kernel<<<256, 256, 0, stream>>>(static_cast<uint4*>(p), kStaticScratchBytes / 16);
    if ((e = hipGetLastError()) != hipSuccess) return hip_status(e);
    st.ptr[dev] = static_cast<char*>(p);
  }
  *out = st.ptr[dev];
  return FL_OK;
}

}  // namespace

extern "C" {

int fl_scan_forward_ex(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                       int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                       const float* ti, const float* gamma, const float* state_in,
                       float* state_out, void* read, int read_dtype, void* workspace,
                       size_t workspace_bytes_given, int algo, void* stream) {
  return scan_impl(raw, raw_dtype, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma, state_in,
                   state_out, read, read_dtype, workspace, workspace_bytes_given, algo,
                   NormArgs{nullptr, 0.f}, stream);
}

int fl_scan_norm_forward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                         int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                         const float* ti, const float* gamma, const float* state_in,
                         float* state_out, const float* norm_weight, float eps, void* out,
                         int out_dtype, void* workspace, size_t workspace_bytes_given,
                         void* stream) {
  if (norm_weight == nullptr) return FL_ERR_INVALID_ARGUMENT;
  return scan_impl(raw, raw_dtype, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma, state_in,
                   state_out, out, out_dtype, workspace, workspace_bytes_given, FL_ALGO_LOOKBACK,
                   NormArgs{norm_weight, eps}, stream);
}

int fl_scan_forward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                    int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
                    const float* gamma, const float* state_in, float* state_out, void* read,
                    int read_dtype, void* workspace, size_t workspace_bytes_given, void* stream) {
  return fl_scan_forward_ex(raw, raw_dtype, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma,
                            state_in, state_out, read, read_dtype, workspace,
                            workspace_bytes_given, FL_ALGO_AUTO, stream);
}

int fl_scan_forward_static(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                           int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                           const float* ti, const float* gamma, const float* state_in,
                           float* state_out, void* read, int read_dtype, void* stream) {
  constexpr LookbackTiling tl = kLookbackTilings[0];
  if (B > 0 && T > 0 && C > 0 &&
      B * cdiv(C, 64 * tl.k) * cdiv(T, (int64_t)tl.l * tl.w) > (int64_t)kStaticMaxTiles)
    return FL_ERR_WORKSPACE;  // beyond what the static scratch holds
  char* base = nullptr;
  const int rc = static_scratch(static_cast<hipStream_t>(stream), &base);
  if (rc != FL_OK) return rc;
  const WsRegions rg{reinterpret_cast<LookbackHeader*>(base),
                     reinterpret_cast<uint32_t*>(base + kStaticStatusOff),
                     reinterpret_cast<uint64_t*>(base + kStaticDataOff), nullptr,
                     clear_span_after_header(base, kStaticScratchBytes)};
  return scan_impl(raw, raw_dtype, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma, state_in,
                   state_out, read, read_dtype, nullptr, 0, FL_ALGO_AUTO, NormArgs{nullptr, 0.f},
                   stream, &rg);
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

int fl_decode_norm_step(const void* raw_t, int raw_dtype, int64_t B, int64_t C,
                        int64_t raw_stride_b, const float* tr, const float* ti,
                        const float* gamma, float* state, const float* norm_weight, float eps,
                        void* out_t, int out_dtype, void* stream) {
  if (raw_dtype != FL_DTYPE_F32 && raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (out_dtype != FL_DTYPE_F32 && out_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (B <= 0 || C <= 0 || B > kMaxB || C > kMaxC) return FL_ERR_INVALID_ARGUMENT;
  if (raw_stride_b < 3 * C) return FL_ERR_INVALID_ARGUMENT;
  if (!raw_t || !tr || !ti || !gamma || !state || !norm_weight || !out_t)
    return FL_ERR_INVALID_ARGUMENT;
  if (!(eps >= 0.f)) return FL_ERR_INVALID_ARGUMENT;
  const size_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  const size_t osz = out_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (!aligned(raw_t, esz) || !aligned(state, 4) || !aligned(out_t, osz) ||
      !aligned(norm_weight, 4) || !aligned(tr, 4) || !aligned(ti, 4) || !aligned(gamma, 4))
    return FL_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float inv_n = (float)(1.0 / (4.0 * (double)C));
#define FL_DN1(R, O, N)                                                                         \
  fl_decode_norm_kernel<R, O, N><<<(unsigned)B, kDecodeNormThreads, 0, s>>>(                     \
      static_cast<const R*>(raw_t), raw_stride_b, (int)C, tr, ti, gamma, state, norm_weight, eps, \
      inv_n, static_cast<O*>(out_t));                                                            \
  return hip_status(hipGetLastError());
#define FL_DN(R, O)                                                                             \
  if (C <= kDecodeNormThreads) { FL_DN1(R, O, 1) }                                              \
  if (C <= 2 * kDecodeNormThreads) { FL_DN1(R, O, 2) }                                          \
  if (C <= 4 * kDecodeNormThreads) { FL_DN1(R, O, 4) }                                          \
  if (C <= 8 * kDecodeNormThreads) { FL_DN1(R, O, 8) }                                          \
  FL_DN1(R, O, 0)
  const bool raw16 = raw_dtype == FL_DTYPE_BF16, out16 = out_dtype == FL_DTYPE_BF16;
  if (raw16 && out16) { FL_DN(bf16_bits, bf16_bits) }
  if (raw16) { FL_DN(bf16_bits, float) }
  if (out16) { FL_DN(float, bf16_bits) }
  FL_DN(float, float)
#undef FL_DN
#undef FL_DN1
}

size_t fl_scan_backward_workspace_bytes(int64_t B, int64_t T, int64_t C) {
  if (B <= 0 || T <= 0 || C <= 0) return 0;
  return bwd_layout(B, T, C).bytes;
}

int fl_scan_backward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                     int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
                     const float* gamma, const float* state_in, const float* read,
                     const float* grad_read, const float* grad_state_out, void* grad_raw,
                     int grad_raw_dtype, float* grad_tr, float* grad_ti, float* grad_gamma,
                     float* grad_state_in, void* workspace, size_t workspace_bytes_given,
                     void* stream) {
  if (raw_dtype != FL_DTYPE_F32 && raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (grad_raw_dtype != FL_DTYPE_F32 && grad_raw_dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (B <= 0 || T <= 0 || C <= 0 || B > kMaxB || C > kMaxC || T > kMaxT)
    return FL_ERR_INVALID_ARGUMENT;
  if (raw_stride_t < 3 * C || raw_stride_b < 0) return FL_ERR_INVALID_ARGUMENT;
  if (B > 1 && raw_stride_b < (T - 1) * raw_stride_t + 3 * C) return FL_ERR_INVALID_ARGUMENT;
  const int64_t esz = raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  const int64_t gsz = grad_raw_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (raw_stride_t * esz > kMaxRowBytes || 4 * C * 4 > kMaxRowBytes) return FL_ERR_INVALID_ARGUMENT;
  if (B * cdiv(T, 32) * cdiv(C, 64) >= ((int64_t)1 << 31)) return FL_ERR_INVALID_ARGUMENT;
  if (!raw || !tr || !ti || !gamma || !read || !grad_read || !grad_raw || !grad_tr || !grad_ti ||
      !grad_gamma)
    return FL_ERR_INVALID_ARGUMENT;
  if (!workspace || workspace_bytes_given < bwd_layout(B, T, C).bytes) return FL_ERR_WORKSPACE;
  if (!aligned(raw, esz) || !aligned(grad_raw, gsz) || !aligned(workspace, 256) ||
      !aligned(read, 4) || !aligned(grad_read, 4) || (state_in && !aligned(state_in, 4)) ||
      (grad_state_out && !aligned(grad_state_out, 4)) || (grad_state_in && !aligned(grad_state_in, 4)))
    return FL_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define FL_BW(R, G)                                                                              \
  return launch_backward<R, G>(raw, B, T, C, raw_stride_b, raw_stride_t, tr, ti, gamma, state_in, \
                               read, grad_read, grad_state_out, grad_raw, grad_tr, grad_ti,       \
                               grad_gamma, grad_state_in, workspace, workspace_bytes_given, s);
  const bool raw16 = raw_dtype == FL_DTYPE_BF16, g16 = grad_raw_dtype == FL_DTYPE_BF16;
  if (raw16 && g16) { FL_BW(bf16_bits, bf16_bits) }
  if (raw16) { FL_BW(bf16_bits, float) }
  if (g16) { FL_BW(float, bf16_bits) }
  FL_BW(float, float)
#undef FL_BW
}

int fl_gate_residual_norm(const void* x, int x_dtype, const void* out, const void* gate_pre,
                          int g_dtype, int64_t rows, int64_t dim, int64_t gate_stride,
                          const float* norm_weight, float eps, void* x_new, void* normed,
                          void* stream) {
  if ((x_dtype != FL_DTYPE_F32 && x_dtype != FL_DTYPE_BF16) ||
      (g_dtype != FL_DTYPE_F32 && g_dtype != FL_DTYPE_BF16))
    return FL_ERR_DTYPE;
  if (rows <= 0 || dim <= 0 || rows > ((int64_t)1 << 31) - 1 || dim > ((int64_t)1 << 24))
    return FL_ERR_INVALID_ARGUMENT;
  if (gate_stride < dim || gate_stride > ((int64_t)1 << 31)) return FL_ERR_INVALID_ARGUMENT;
  if (!x || !out || !gate_pre || !norm_weight || !x_new || !normed || !(eps >= 0.f))
    return FL_ERR_INVALID_ARGUMENT;
  const size_t xs = x_dtype == FL_DTYPE_BF16 ? 2 : 4, gs = g_dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (!aligned(x, xs) || !aligned(x_new, xs) || !aligned(normed, xs) || !aligned(out, gs) ||
      !aligned(gate_pre, gs) || !aligned(norm_weight, 4))
    return FL_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float inv = (float)(1.0 / (double)dim);
#define FL_GRN1(X, G, N)                                                                        \
  fl_gate_residual_norm_kernel<X, G, N><<<(unsigned)rows, kTailThreads, 0, s>>>(                \
      static_cast<const X*>(x), static_cast<const G*>(out), static_cast<const G*>(gate_pre),    \
      gate_stride, (int)dim, norm_weight, eps, inv, static_cast<X*>(x_new),                     \
      static_cast<X*>(normed));                                                                 \
  return hip_status(hipGetLastError());
#define FL_GRN(X, G)                                                                            \
  if (dim <= kTailThreads) { FL_GRN1(X, G, 1) }                                                 \
  if (dim <= 2 * kTailThreads) { FL_GRN1(X, G, 2) }                                             \
  if (dim <= 4 * kTailThreads) { FL_GRN1(X, G, 4) }                                             \
  if (dim <= 8 * kTailThreads) { FL_GRN1(X, G, 8) }                                             \
  FL_GRN1(X, G, 0)
  const bool x16 = x_dtype == FL_DTYPE_BF16, g16 = g_dtype == FL_DTYPE_BF16;
  if (x16 && g16) { FL_GRN(bf16_bits, bf16_bits) }
  if (x16) { FL_GRN(bf16_bits, float) }
  if (g16) { FL_GRN(float, bf16_bits) }
  FL_GRN(float, float)
#undef FL_GRN
#undef FL_GRN1
}

int fl_swiglu(const void* gate_up, int dtype, int64_t rows, int64_t hidden, void* out,
              void* stream) {
  if (dtype != FL_DTYPE_F32 && dtype != FL_DTYPE_BF16) return FL_ERR_DTYPE;
  if (rows <= 0 || hidden <= 0 || hidden > ((int64_t)1 << 30)) return FL_ERR_INVALID_ARGUMENT;
  if (!gate_up || !out) return FL_ERR_INVALID_ARGUMENT;
  const size_t es = dtype == FL_DTYPE_BF16 ? 2 : 4;
  if (!aligned(gate_up, es) || !aligned(out, es)) return FL_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n = rows * hidden;
  const unsigned blocks = (unsigned)(cdiv(n, 256) < 4096 ? cdiv(n, 256) : 4096);
  if (dtype == FL_DTYPE_BF16)
    fl_swiglu_kernel<bf16_bits><<<blocks, 256, 0, s>>>(static_cast<const bf16_bits*>(gate_up), rows,
                                                        (int)hidden, static_cast<bf16_bits*>(out));
  else
    fl_swiglu_kernel<float><<<blocks, 256, 0, s>>>(static_cast<const float*>(gate_up), rows,
                                                    (int)hidden, static_cast<float*>(out));
  return hip_status(hipGetLastError());
}

int fl_boundary_scan(const float* a, const float* drive, int64_t B, int64_t T, int64_t R,
                     const float* state_in, float* state_out, float* out, void* stream) {
  if (B <= 0 || T <= 0 || R <= 0 || B > kMaxB || R > kMaxC || T > kMaxT)
    return FL_ERR_INVALID_ARGUMENT;
  if (T * R >= ((int64_t)1 << 40)) return FL_ERR_INVALID_ARGUMENT;
  if (!a || !drive || !out) return FL_ERR_INVALID_ARGUMENT;
  if (!aligned(a, 4) || !aligned(drive, 4) || !aligned(out, 4) ||
      (state_in && !aligned(state_in, 4)) || (state_out && !aligned(state_out, 4)))
    return FL_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)B, (unsigned)cdiv(R, 64));
  fl_boundary_scan_kernel<<<grid, kBoundaryWaves * 64, 0, static_cast<hipStream_t>(stream)>>>(
      a, drive, (int)T, (int)R, state_in, state_out, out);
  return hip_status(hipGetLastError());
}

}  // extern "C"
