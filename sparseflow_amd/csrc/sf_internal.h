// Internal declarations shared by the prescan / conv translation units and
// the C ABI.  gfx950 only: wave64, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <atomic>

#include "sparseflow.h"

namespace sf {

constexpr int kWave = 64;
constexpr int kMaxLdsBytes = 160 * 1024;

// ---------------------------------------------------------------------------
// Pack plan: how Stage 1a tiles the pixel axis.  A "chunk" is the run of
// consecutive pixels (within one frame) that one wavefront covers; the
// non-binary flag array has one word per chunk.  The plan depends on the
// shape only, so Stage 2 can recompute it to index the flags.
// ---------------------------------------------------------------------------
struct PackPlan {
  int vec;                   // pixels per lane (4, 2 or 1)
  int chunk;                 // pixels per chunk = 64 * vec
  int csplit;                // waves sharing one chunk (split over words)
  int cwp;                   // bitmap words per pixel
  int64_t chunks_per_frame;  // ceil(h*w / chunk)
  int64_t total_chunks;      // n * chunks_per_frame
};

PackPlan make_pack_plan(int64_t n, int c, int h, int w);
int words_per_pixel(int c);

// ---------------------------------------------------------------------------
// Kernel argument blocks (passed by value).
// ---------------------------------------------------------------------------
struct PackArgs {
  const void* x;
  uint32_t* bits;
  uint32_t* flags;
  int64_t n;
  int c, hw, cwp, csplit, vec;
  int64_t chunks_per_frame, total_chunks;
  float cutoff;
  int planar;  // 1: words as [frame][cwp][hw] (word planes), 0: [frame][hw][cwp]
};

struct TilesArgs {
  const uint32_t* bits;
  uint32_t* ch_mask;
  int32_t* ch_count;
  int32_t* ch_list;
  int32_t* ag_mask;
  int32_t* tile_class;
  int64_t n, ntiles;
  int c, cwp, h_in, w_in, h_out, w_out, k, s, p;
  int th, tw, gh, gw, group_size, ngroups;
};

struct ConvArgs {
  const uint32_t* bits;
  const uint32_t* flags;
  const void* x;
  const float* wt;
  const float* bias;
  void* y;             // conv output, or spikes for the fused LIF kernel
  float* v_out;        // fused LIF only
  const float* v_init; // fused LIF only (nullable)
  int64_t n;           // frames of y (conv) / batch N (LIF)
  int64_t total_groups;
  int c_in, h_in, w_in, c_out, h_out, w_out, k, s, p, cwp;
  // Bitmap word w of input pixel q of a frame sits at q * bm_ps + w * bm_ws
  // words from the frame's start: (cwp, 1) for the [hw][cwp] layout of
  // sf_prescan_pack, (1, hw_in) for word planes (the kernels that load one
  // word of 64 pixels at a time: px3 and rows_kc).
  int bm_ps, bm_ws;
  int hw_in, hw_out, groups_per_frame;
  int chunk;                 // flag chunk (pixels)
  int64_t chunks_per_frame;
  int cap;                   // entry-list capacity per wave
  int fl;                    // pixels per staging flush
  int wave_lds;              // LDS bytes per wave
  int waves_per_block;
  int T;                     // fused LIF: time steps
  float tau, v_th, v_reset;
  int hard_reset, decay_input;
};

// Launchers (return hipError_t as int).
int launch_pack(const PackArgs& a, int dtype, hipStream_t stream);
int launch_tiles(const TilesArgs& a, hipStream_t stream);
int launch_conv(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);
int launch_conv_lif(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Row-band Stage 2 from the bitmap (3x3 s1, C_in <= 64, frame width 32),
// lane = output channel.
bool band_applicable(const ConvArgs& a);
int launch_conv_band(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// The same walk with Stage 1 fused in (3x3 s1, C_in <= 64, frame width 32):
// reads x directly (a.bits / a.flags unused); bit = |x| >= cutoff.
bool rows_fused_applicable(const ConvArgs& a);
int launch_conv_rows_fused(const ConvArgs& a, int in_dtype, int out_dtype, float cutoff, hipStream_t stream);

// K-chunked row-tile Stage 2 (3x3 s1, any C_in, frame width 28 or 14).
bool rows_kc_applicable(const ConvArgs& a);
int launch_conv_rows_kc(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Flat-tile Stage 2 for 1x1 stride-1 convolutions (any C_in, C_out % 4 == 0).
bool flat_applicable(const ConvArgs& a);
int launch_conv_flat(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Pixel-tile Stage 2 for 3x3 convolutions (stride 1 or 2, C_out % 4 == 0).
bool px3_applicable(const ConvArgs& a);
// The weights stay resident in LDS for the whole launch (C_in <= 128).
bool px3_resident(const ConvArgs& a);
int launch_conv_px3(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);
// Matrix-core Stage 2 for 3x3 layers with a reduction of at most 32
// (C_in * 9 <= 32, f32 input): the whole K is one dense tile.
bool mfma_conv_applicable(const ConvArgs& a);
int launch_conv_mfma(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);
// Dense-tile branch of the streamed pixel-tile kernel (k_conv_px3s) and of
// the row kernel (k_conv_rows_kc): tiles whose first chunk is dense go to a
// queue (per 64-output-channel group, a run of at most 64 output pixels of
// the flattened (frame, pixel) axis: its first pixel and its length) and are
// computed on the matrix cores by launch_conv_dense_mfma, launched right
// after on the same stream; its last workgroup clears the counts.  One queue
// slot per stream (library-owned static device memory); dense_queue_for
// returns the stream's slot, or NULL when every slot is taken (then nothing
// is deferred).
constexpr int kDenseQueueSlots = 8;
constexpr int kDenseQueueGroups = 32;   // C_out <= 2048
constexpr int kDenseQueueCap = 4096;    // runs per group; more are walked
struct DenseQueue {
  uint32_t count[kDenseQueueGroups];
  uint32_t done;
  uint32_t pad[31];
  uint32_t start[kDenseQueueGroups][kDenseQueueCap];  // first output pixel of the run
  uint8_t npx[kDenseQueueGroups][kDenseQueueCap];     // its pixels (1 .. 64)
};
DenseQueue* dense_queue_for(hipStream_t stream);
// Looks up the queue array's device address on the current GPU (once; it
// may load the code object there).  hipError_t as int.
int dense_queue_prepare();
int launch_conv_dense_mfma(const ConvArgs& a, DenseQueue* dq, int out_dtype, hipStream_t stream);
// Deferral test on a wave-tile's first chunk: some pixel of it has at least
// kDenseLaneSpikes active (tap, channel) pairs there.  The walk lasts as long
// as the busiest pixel's count in every chunk, while the matrix cores' cost
// is fixed (about that of a 16-round chunk walk); i.i.d. input at 1%
// density has 2.9 per pixel on average and a tile passes with probability
// ~6e-5, at 3% most tiles pass, and so does any tile with a hot pixel.
constexpr int kDenseLaneSpikes = 16;

// Fused conv + multi-step LIF on the pixel-tile formulation (3x3 s1; same
// applicability as px3_applicable with stride 1).
int launch_conv_lif_px3(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Fused 1x1 s1 conv + multi-step LIF on the flat pixel-tile kernel (a: n =
// samples, T steps, bits of the T*n input frames); x2: optional residual
// (conv-output layout, x's dtype) added into each step's current; out_bits /
// out_flags: optional spike map of the output (out_cwp words per pixel,
// pixel-major or as word planes when out_planes != 0; flag chunks of
// out_chunk pixels, out_cpf per frame); res_bits: optional binary residual
// as its pixel-major spike map, read instead of x2.
int launch_conv_lif_flat(const ConvArgs& a, int in_dtype, int out_dtype, const void* x2, const uint32_t* res_bits,
                         uint32_t* out_bits, uint32_t* out_flags, int out_cwp, int out_planes, int out_chunk,
                         int64_t out_cpf, hipStream_t stream);

// Standalone multi-step LIF over T steps of n x c x hw neurons (x2: optional
// second input summed into the current; bits: optional spike map output
// with cwp words per pixel, pixel-major or as word planes (planes != 0),
// with its nflags chunk flags cleared).
// Spike max pooling from a spike map (at most kSpikePoolMaxWords words, 256
// channels, per pixel).
constexpr int kSpikePoolMaxWords = 8;
int launch_spike_maxpool(const uint32_t* bits, int64_t n, int c, int h_in, int w_in, int h_out, int w_out, int k,
                         int st, int pd, int cwp, int out_dtype, void* y, uint32_t* out_bits, hipStream_t stream);
int launch_lif_multistep(const void* x, const void* x2, int in_dtype, int T, int64_t n, int c, int64_t hw, float tau,
                         float v_th, float v_reset, int hard_reset, int decay_input, const float* v_init, void* spikes,
                         int out_dtype, float* v_out, uint32_t* bits, int cwp, int planes, uint32_t* flags,
                         int64_t nflags, hipStream_t stream);

// Sparse linear (row-major x [m, k], weight wt [k, c_out]): row prescan and
// the flat lane = row Stage 2.  Bitmap words per row: ceil(k/32), rounded up
// to a multiple of 4 beyond two words; one flag word per kLinearRowChunk rows.
constexpr int kLinearRowChunk = 16;
int linear_words_per_row(int k);
int launch_pack_rows(const PackArgs& a, int dtype, hipStream_t stream);
// a: n = 1, hw_in = h_in = h_out = m, w = 1, c_in = k, cwp, chunk =
// kLinearRowChunk, chunks_per_frame = row chunks; y is [m, c_out].
int launch_linear_flat(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Sparse batched matmul C[b] = A[b] @ B[b] (A [batches, m, k] contiguous,
// B through strides, C [batches, m, n] contiguous).
struct BmmArgs {
  const void* a;
  const void* b;
  void* c;
  int64_t batches;
  int m, k, n;
  int64_t b_stride_batch, b_stride_k, b_stride_n;  // elements
  int ncb;                                          // column blocks (set by the launcher)
  float cutoff;
  float alpha;                                      // output scale
};
constexpr int kBmmLdsBytes = 64 * 1024;  // staged B block per workgroup
// Columns per block / 64 (4, 2 or 1) for a k x n B, or 0 when even a
// 64-column block of k rows exceeds the LDS budget.
int bmm_column_blocks(int k, int n);
int launch_bmm(const BmmArgs& a, int in_dtype, int out_dtype, hipStream_t stream);
// The same product on the matrix cores (A's rows dense enough that every
// 32-wide K slice of a 16-row tile is live): k <= 256 and B's bf16 hi + lo
// copy within the LDS budget.
bool bmm_mfma_supported(int k, int n);
int launch_bmm_mfma(const BmmArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Sparse Linear on MFMA: x [m, k] row-major, W split into bf16 hi / lo
// [c_out][kp] (k contiguous, kp = k rounded up to 32, zero padded).
struct LinMfmaArgs {
  const void* x;
  const uint16_t* wh;  // bf16 bit patterns
  const uint16_t* wl;
  const float* bias;
  void* y;
  int64_t m;
  int k, kp, c_out;
  float cutoff;  // elements with |x| < cutoff count as zero
};
int linear_mfma_max_kp();
int launch_linear_mfma(const LinMfmaArgs& a, int in_dtype, int out_dtype, hipStream_t stream);
// The same product over sf_linear_prescan's row bitmap (cwp words per row)
// and its non-binary flags (one per kLinearRowChunk rows).
int launch_linear_bits_mfma(const LinMfmaArgs& a, const uint32_t* bits, const uint32_t* flags, int cwp, int in_dtype,
                            int out_dtype, hipStream_t stream);

// Fused spike attention core y = (q @ k^T * scale) @ v = q @ (k^T v) * scale
// per (frame, head); element (tb, m, h, d) at tb*s_tb + m*s_m + h*s_h + d.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* y;
  int64_t tb;
  int s, h, d;
  int64_t s_tb, s_m, s_h;  // q / k / v strides (elements)
  int64_t y_tb, y_m, y_h;  // y strides
  float scale, cutoff;
};
size_t attn_lds_bytes(int s, int d);
int launch_spike_attn(const AttnArgs& a, int in_dtype, int out_dtype, hipStream_t stream);

// Raise kernel K's dynamic-LDS ceiling to `bytes` (the default limit is
// 64 KB) once per device and process.  Thread-safe: two first calls racing
// set the same attribute twice, which is harmless; a failure is returned and
// the next call tries again.
template <auto K>
int set_lds_limit_once(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return (int)hipSuccess;
  const hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void*>(K), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return (int)e;
}

// Conv launch geometry shared by the ABI (workspace checks) and launchers.
void conv_geometry(ConvArgs& a, bool lif);

// Per-kernel event timing hooks used by the launchers.
void timing_begin(int kernel_id, hipStream_t stream);
void timing_end(int kernel_id, hipStream_t stream);
enum KernelId { K_PACK = 0, K_TILES = 1, K_CONV = 2, K_LIF = 3, K_ROWS = 4, K_ROWS_KC = 5, K_FLAT = 6, K_PX3 = 7, K_LIF_PX3 = 8, K_LIF_MS = 9, K_PACK_ROWS = 10, K_LINEAR = 11, K_BMM = 12, K_ATTN = 13, K_LINEAR_MFMA = 14, K_BMM_MFMA = 15, K_LIF_FLAT = 16, K_MFMA_CONV = 17, K_ROWS_FUSED = 18, K_DENSE_MFMA = 19, K_COUNT = 20 };

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC__)

// Order this wavefront's LDS traffic: writes issued before the call are
// visible to reads issued after it by any lane of the same wavefront.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) {
  return __bfloat162float(v);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
  return __float2bfloat16(v);
}

// Inclusive prefix sum across the 64 lanes of a wavefront.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    int t = __shfl_up(v, off, kWave);
    if (lane >= off) v += t;
  }
  return v;
}

#endif

}  // namespace sf
