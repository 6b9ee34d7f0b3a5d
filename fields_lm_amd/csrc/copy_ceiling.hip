// copy_ceiling.hip — measurement kernels for bench.py (not part of the C ABI of fields_amd.h):
// what the Field scan's memory traffic alone costs on the device, without its arithmetic or its
// look-back, so that the scan's time can be read against the time of its own access pattern.
//
//   fl_bench_tile_copy    the scan's LDS-staged access pattern exactly: tiles of 64 channels x 128
//                         rows, one 512-thread block per tile (8 waves x 16 rows), the same
//                         block -> tile order (the channel tiles of a row group on one XCD), raw
//                         rows loaded with 16-byte loads that write LDS, two blocks per CU, and
//                         the 4 output planes written with 16-byte non-temporal stores; the stored
//                         values are the raw values widened (fp32) or copied (bf16)
//   fl_bench_stream_copy  a streaming copy of the same bytes: 16-byte loads of `in_bytes`,
//                         16-byte non-temporal stores of `out_bytes`, grid-stride
//   fl_bench_device_delay one wave that sleeps until the constant-rate wall clock has advanced by a
//                         given number of ticks, queued before a timed loop's start event so that
//                         the host has its first launches queued when the device reaches it
//   fl_bench_occupy       `blocks` blocks of 1024 threads holding 112 KB of LDS each (so no scan
//                         tile block fits beside one on its CU), each sleeping on the wall clock
//                         for a given time: CUs held by another stream's bounded work, the
//                         contention under which the tests run the scan's block-order launches
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kBufDword3 = 0x00020000u;
constexpr int kNt = 2;  // buffer store cache policy: nt

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufDword3);
}

// block i -> tile (the scan's xcd_grouped_ticket): within each window of 8 row groups, the blocks
// of one XCD (block i runs on XCD i mod 8) take the channel tiles of one row group
__device__ __forceinline__ uint32_t grouped_tile(uint32_t i, uint32_t n_ctiles, uint32_t n_tiles) {
  const uint32_t win = 8u * n_ctiles;
  if (win > 256u) return i;
  const uint32_t w = i / win, u = i - w * win;
  if ((w + 1u) * win > n_tiles) return i;
  return w * win + (u & 7u) * n_ctiles + (u >> 3);
}

// raw bf16 [B, T, 3C] (rows of 3C), out [B, T, 4C] of OSZ-byte elements; T % 128 == 0, C % 64 == 0
template <int OSZ>
__global__ __launch_bounds__(512, 2) void tile_copy_kernel(const uint16_t* __restrict__ raw,
                                                           void* __restrict__ out, int T, int C,
                                                           int n_ctiles, int n_chunks) {
  constexpr int CT = 64, TC = 128, L = 16;
  __shared__ __align__(16) uint16_t s_io[3 * TC * CT];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t n_tiles = gridDim.x;
  const uint32_t n_chains = n_tiles / (uint32_t)n_chunks;
  const uint32_t tile = grouped_tile(blockIdx.x, (uint32_t)n_ctiles, n_tiles);
  const int chunk = (int)(tile / n_chains), chain = (int)(tile - (uint32_t)chunk * n_chains);
  const int b = chain / n_ctiles, ctile = chain - b * n_ctiles;
  const int raw_row = 3 * C * 2, out_row = 4 * C * OSZ;
  const rsrc_t r = make_rsrc(raw + ((int64_t)b * T + (int64_t)chunk * TC) * 3 * C, (uint32_t)(TC * raw_row));
  // this wave's rows: 8 rows of one plane per load (lane = 8 * row + 16-byte piece)
  const int vo = ctile * CT * 2 + (lane >> 3) * raw_row + (lane & 7) * 16;
#pragma unroll
  for (int q = 0; q < 3 * (L / 8); ++q) {
    const int plane = q / (L / 8), r0 = wave * L + (q % (L / 8)) * 8;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)&s_io[(plane * TC + r0) * CT], 16, vo,
        r0 * raw_row + plane * C * 2, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the wave reads only the rows it loaded itself
  const rsrc_t w = make_rsrc(static_cast<char*>(out) + ((int64_t)b * T + (int64_t)chunk * TC) * out_row,
                             (uint32_t)(TC * out_row));
  constexpr int per_rp = CT * OSZ / 16;  // lanes per row-plane
  constexpr int rp_per = 64 / per_rp;    // row-planes per store
#pragma unroll
  for (int i = 0; i < 4 * L / rp_per; ++i) {
    const int rp = i * rp_per + lane / per_rp, row = wave * L + rp / 4, plane = rp % 4;
    const int piece = lane % per_rp;
    const uint16_t* src = &s_io[((plane % 3) * TC + row) * CT];
    u32x4 v;
    if constexpr (OSZ == 4) {  // 4 channels widened
      const uint2 h = *reinterpret_cast<const uint2*>(src + 4 * piece);
      v.x = h.x << 16; v.y = h.x & 0xffff0000u; v.z = h.y << 16; v.w = h.y & 0xffff0000u;
    } else {  // 8 channels
      v = *reinterpret_cast<const u32x4*>(src + 8 * piece);
    }
    const int off = row * out_row + plane * C * OSZ + ctile * CT * OSZ + 16 * piece;
    __builtin_amdgcn_raw_buffer_store_b128(v, w, off, 0, kNt);
  }
}

__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                          u32x4* __restrict__ dst, size_t n_in,
                                                          size_t n_out) {
  const size_t n = n_in > n_out ? n_in : n_out;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const u32x4 v = i < n_in ? src[i] : (u32x4){(uint32_t)i, 1u, 2u, 3u};
    if (i < n_out) __builtin_nontemporal_store(v, &dst[i]);
  }
}

// returns once wall_clock64() has advanced by `ticks` (a monotonic constant-rate counter)
__global__ __launch_bounds__(64) void delay_kernel(uint64_t ticks) {
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// One CU's worth of LDS held for `ticks` of the wall clock (bounded: every block exits).
constexpr int kOccupyLdsFloats = 112 * 1024 / 4;
__global__ __launch_bounds__(1024) void occupy_kernel(uint64_t ticks, float* sink) {
  __shared__ float hold[kOccupyLdsFloats];
  for (int i = threadIdx.x; i < kOccupyLdsFloats; i += 1024) hold[i] = (float)i;
  __syncthreads();
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
  // a value read back from the array, so that the compiler keeps it; never true
  if (hold[(threadIdx.x * 37) % kOccupyLdsFloats] < -1.0f) sink[threadIdx.x] = hold[threadIdx.x];
}

int wall_ticks(double us, uint64_t* ticks) {
  int dev = 0, khz = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return (int)e;
  if (khz <= 0) return 1;
  *ticks = (uint64_t)(us * (double)khz / 1000.0);
  return 0;
}

}  // namespace

extern "C" {

// The scan's tile pattern for raw bf16 [B, T, 3C] -> out [B, T, 4C] (out_bytes_per_elem 4 or 2).
// Returns 1 for shapes outside the pattern (T % 128, C % 64, buffer alignment), else the HIP status.
int fl_bench_tile_copy(const void* raw, void* out, int64_t B, int64_t T, int64_t C,
                       int out_bytes_per_elem, void* stream) {
  if (B <= 0 || T <= 0 || C <= 0 || T % 128 != 0 || C % 64 != 0) return 1;
  if ((uintptr_t)raw % 16 != 0 || (uintptr_t)out % 16 != 0) return 1;
  if (128 * 4 * C * out_bytes_per_elem >= ((int64_t)1 << 31)) return 1;
  const int n_ctiles = (int)(C / 64), n_chunks = (int)(T / 128);
  const unsigned grid = (unsigned)(B * n_ctiles * n_chunks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* r = static_cast<const uint16_t*>(raw);
  if (out_bytes_per_elem == 4)
    tile_copy_kernel<4><<<grid, 512, 0, s>>>(r, out, (int)T, (int)C, n_ctiles, n_chunks);
  else if (out_bytes_per_elem == 2)
    tile_copy_kernel<2><<<grid, 512, 0, s>>>(r, out, (int)T, (int)C, n_ctiles, n_chunks);
  else
    return 1;
  return (int)hipGetLastError();
}

// Streaming copy: reads in_bytes from src and writes out_bytes to dst (both multiples of 16,
// 16-byte aligned).
int fl_bench_stream_copy(const void* src, void* dst, size_t in_bytes, size_t out_bytes, void* stream) {
  if (in_bytes % 16 != 0 || out_bytes % 16 != 0) return 1;
  if ((uintptr_t)src % 16 != 0 || (uintptr_t)dst % 16 != 0) return 1;
  stream_copy_kernel<<<2048, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), in_bytes / 16, out_bytes / 16);
  return (int)hipGetLastError();
}

// Queues ~`us` microseconds of device time (one wave) on `stream`; at most 10 ms.
int fl_bench_device_delay(double us, void* stream) {
  if (!(us >= 0.0) || us > 10000.0) return 1;
  uint64_t ticks = 0;
  const int rc = wall_ticks(us, &ticks);
  if (rc != 0) return rc;
  delay_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(ticks);
  return (int)hipGetLastError();
}

// Queues `blocks` (1..256) blocks that each hold one CU's LDS for ~`us` microseconds (at most
// 10 ms) on `stream`. `sink` is a device buffer of 1024 floats that is never written in practice.
int fl_bench_occupy(int blocks, double us, void* sink, void* stream) {
  if (blocks < 1 || blocks > 256 || !(us >= 0.0) || us > 10000.0 || sink == nullptr) return 1;
  uint64_t ticks = 0;
  const int rc = wall_ticks(us, &ticks);
  if (rc != 0) return rc;
  occupy_kernel<<<blocks, 1024, 0, static_cast<hipStream_t>(stream)>>>(ticks, static_cast<float*>(sink));
  return (int)hipGetLastError();
}

}  // extern "C"
