// Stage 2 for 3x3 convolutions (stride 1 or 2, padding 1): 64-pixel output
// tiles, lane = output pixel.
//
// One wavefront owns 64 consecutive output pixels (a flat run of the
// h_out*w_out plane) for a slice of 64 or 32 output channels: lane = output
// pixel, one accumulator register per output channel.  For a run of input
// channels each lane loads the bitmap words of its 9 input taps (0 outside
// the frame) and walks its own spikes in (tap, ci) order with a per-lane
// cursor: a divergent loop whose round count is the busiest pixel's spike
// count.  Every spike adds weight row (ci, tap) -- the slice's output
// channels, read from LDS as 16-byte pieces -- to the lane's accumulators.
// The finished tile is stored one output channel per instruction (64
// consecutive pixels = one 256-byte run of the channel plane).
//
// Variants (launch_px3_conv picks one):
//  k_conv_px3w  C_in <= 128: every weight row of the slice resident in LDS
//               (64 input channels x 64 output channels, rows padded to 272
//               bytes, or 128 x 32 with 128-byte rows, pieces swizzled), the
//               spikes walked 64 channels at a time (64-bit masks); also the
//               fused conv-LIF for C_in <= 128.
//  k_conv_px3s  C_in > 128: 32-channel chunks of 64 output channels streamed
//               through two LDS buffers (chunk c+1 arrives while chunk c is
//               walked), tiles of the flattened (frame, pixel) axis.
//  k_conv_px3   the per-frame-tile form (32-channel chunks, resident or
//               streamed): the fused conv-LIF for C_in > 128 and the
//               fallback for tensors beyond one buffer resource.
// The persistent forms size their workgroups so that every CU makes the same
// number of passes.  The bitmap words are read through two strides, so the
// same kernels take the [hw][cwp] words of sf_prescan_pack and the word
// planes sf_conv2d_forward packs for them.
//
// Output element (co, oh, ow) = bias[co] + its active taps summed by one lane
// in (channel block, tap, ci) order: deterministic from run to run.
// Replaces the reference's sparse_conv3x3s1_nhwc_kernel_8x8/8x16 and
// sparse_conv3x3s2 kernels (Kernels/conv2d.py:564-886) for these shapes.
#include <type_traits>

#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kPx3Ch = 32;               // input channels per chunk (one bitmap word)
constexpr int kPx3Rows = kPx3Ch * 9;     // weight rows per chunk

// LDS layout of a chunk for a workgroup slice of CO output channels.
//  CO = 64: rows of 16 pieces (16 bytes = 4 channels) padded to 17 pieces
//           (272 bytes), read at immediate offsets.
//  CO = 32: rows of 8 pieces (128 bytes), piece s of row r stored at
//           position s ^ ((r >> 1) & 7) so that lanes reading different rows
//           spread over the banks without padding (the whole 128-channel
//           config-4 layer stays resident).
template <int CO>
struct Px3Layout {
  static constexpr int pieces = CO / 4;                         // logical pieces per row
  static constexpr int stride = CO == 64 ? 17 : pieces;         // pieces per row in LDS
  static constexpr int xmask = CO == 64 ? 0 : (pieces >= 8 ? 7 : pieces - 1);  // piece swizzle
  static constexpr int units = (kPx3Rows * stride + 63) / 64;   // 1 KB load units per chunk
  static constexpr int chunk_bytes = units * 1024;
  // Chunks that fit at once (1 KB of the LDS is left to static arrays).
  static constexpr int resident_chunks = (kMaxLdsBytes - 1024) / chunk_bytes;
};

// Direct-to-LDS loads of weight chunk c (output channels co0 .. co0+CO-1).
// The chunk is an array of 16-byte positions; unit u fills positions
// 64 u .. 64 u + 63, lane l position 64 u + l.  Pads, rows past C_in and
// channels past C_out read a valid but unrelated address whose values are
// never used.
template <int CO>
__device__ __forceinline__ void load_chunk_px3(char* buf, const float* __restrict__ wt, int c, int krows,
                                               int c_out, int co0, int wave, int lane) {
  typedef Px3Layout<CO> L;
#pragma unroll
  for (int j = 0; j < (L::units + kRowsWaves - 1) / kRowsWaves; ++j) {
    const int u = wave + kRowsWaves * j;
    if (u < L::units) {
      const int pos = u * 64 + lane;
      const int r = pos / L::stride;
      const int q = pos - r * L::stride;
      const int s = CO == 64 ? q : (q ^ ((r >> 1) & L::xmask));  // logical piece stored at position q
      const int row = c * kPx3Rows + r;
      const int col = co0 + 4 * s;
      const float* src =
          (q < L::pieces && r < kPx3Rows && row < krows && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  }
}

// Add the weight row at rowp (piece swizzle key for CO = 32), times xv, to
// the CO accumulators.  WHOLE (CO = 32 kernels with registers to spare, not
// the fused LIF kernels, which use all 128): all eight pieces are read
// before the first FMA, one LDS wait per spike instead of one per pair.
template <int CO, bool WHOLE = false>
__device__ __forceinline__ void px3_add_row_at(float (&acc)[CO], const char* rowp, int key, float xv) {
  typedef Px3Layout<CO> L;
  if constexpr (CO == 32 && WHOLE) {
    float4 v[L::pieces];
#pragma unroll
    for (int s = 0; s < L::pieces; ++s) v[s] = *reinterpret_cast<const float4*>(rowp + ((s << 4) ^ key));
#pragma unroll
    for (int s = 0; s < L::pieces; ++s) {
      acc[4 * s] = fmaf(xv, v[s].x, acc[4 * s]);
      acc[4 * s + 1] = fmaf(xv, v[s].y, acc[4 * s + 1]);
      acc[4 * s + 2] = fmaf(xv, v[s].z, acc[4 * s + 2]);
      acc[4 * s + 3] = fmaf(xv, v[s].w, acc[4 * s + 3]);
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < L::pieces; ++s) {
    // Groups of four pieces: the scheduler may not hoist more than 16
    // loaded registers ahead of their use (the accumulators take CO).
    if (s % 4 == 0) __builtin_amdgcn_sched_barrier(0);
    const float4 v = CO == 64 ? reinterpret_cast<const float4*>(rowp)[s]
                              : *reinterpret_cast<const float4*>(rowp + ((s << 4) ^ key));
    acc[4 * s] = fmaf(xv, v.x, acc[4 * s]);
    acc[4 * s + 1] = fmaf(xv, v.y, acc[4 * s + 1]);
    acc[4 * s + 2] = fmaf(xv, v.z, acc[4 * s + 2]);
    acc[4 * s + 3] = fmaf(xv, v.w, acc[4 * s + 3]);
  }
}

// Add weight row r of the chunk, times xv, to the CO accumulators.
template <int CO, bool WHOLE = false>
__device__ __forceinline__ void px3_add_row(float (&acc)[CO], const char* chunk, int r, float xv) {
  typedef Px3Layout<CO> L;
  px3_add_row_at<CO, WHOLE>(acc, chunk + (r * L::stride) * 16, CO == 64 ? 0 : ((r >> 1) & L::xmask) << 4, xv);
}

// Rows (ci, tap) of a 64-channel chunk (272-byte rows, row ci * 9 + tap):
// the tap's row start is formed once per refill of a lane's word, the
// channel's offset per spike with one 24-bit multiply-add (a chunk spans
// fewer than 2^24 bytes) instead of a full 32-bit multiply of the row index.
constexpr uint32_t kPx3RowBytes = Px3Layout<64>::stride * 16;
__device__ __forceinline__ const char* px3_tap_rows(const char* chunk, int tap) {
  return chunk + __umul24((uint32_t)tap, kPx3RowBytes);
}
__device__ __forceinline__ const char* px3_spike_row(const char* tap_rows, int ci) {
  return tap_rows + __umul24((uint32_t)ci, 9u * kPx3RowBytes);
}
// The tap back from its row start (the multiply-by-x path only: the walk keeps
// one register per lane for the tap, its row start).
__device__ __forceinline__ int px3_rows_tap(const char* chunk, const char* tap_rows) {
  return (int)((uint32_t)(tap_rows - chunk) / kPx3RowBytes);
}

// Word of tap t among the lane's nine: a per-lane 9-way multiplexer on the
// bits of t (eight selects).
__device__ __forceinline__ uint32_t px3_select(const uint32_t (&w)[9], int t) {
  const uint32_t v0 = w[0], v1 = w[1], v2 = w[2], v3 = w[3], v4 = w[4], v5 = w[5], v6 = w[6], v7 = w[7], v8 = w[8];
  const bool b0 = t & 1, b1 = t & 2, b2 = t & 4, b3 = t & 8;
  const uint32_t a0 = b0 ? v1 : v0, a1 = b0 ? v3 : v2;
  const uint32_t a2 = b0 ? v5 : v4, a3 = b0 ? v7 : v6;
  const uint32_t c0 = b1 ? a1 : a0, c1 = b1 ? a3 : a2;
  const uint32_t d0 = b2 ? c1 : c0;
  return b3 ? v8 : d0;
}

// Bitmap word c of each of the lane's nine input taps (0 outside the frame),
// bf = the frame's bitmap (word c of pixel q at q * bm_ps + c * bm_ws).  Raw
// buffer loads over the frame's words: a tap outside the frame gets an
// offset past num_records, which the hardware returns as 0, so no
// instruction has to touch the loaded values until they are used (the next
// chunk's words are requested a whole chunk walk ahead).  With word planes
// (bm_ps = 1) the 64 lanes of a load read one run of neighbouring words;
// with [hw][cwp] words each lane touches its own cache line once cwp >= 8.
__device__ __forceinline__ void px3_load_words(uint32_t (&w)[9], const uint32_t* __restrict__ bf,
                                               const ConvArgs& a, int ih0, int iw0, int c) {
  const uint32_t frame_bytes = (uint32_t)a.hw_in * (uint32_t)a.cwp * 4u;
  const auto rs = buf_rsrc(bf, frame_bytes);
  const uint32_t cofs = (uint32_t)c * (uint32_t)a.bm_ws;
#pragma unroll
  for (int tp = 0; tp < 9; ++tp) {
    const int ih = ih0 + tp / 3, iw = iw0 + tp % 3;
    const bool in = ih >= 0 && ih < a.h_in && iw >= 0 && iw < a.w_in;
    const uint32_t off = in ? ((uint32_t)(ih * a.w_in + iw) * (uint32_t)a.bm_ps + cofs) * 4u : 0x80000000u;
    w[tp] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
  }
}

// Tile t of a wavefront (64 output pixels of one sample): whether this lane
// has an output pixel there, and its sample and the top-left corner of its
// input window.
__device__ __forceinline__ bool px3_tile(const ConvArgs& a, int t, int lane, int total, int tpf, int& sample,
                                         int& ih0, int& iw0) {
  if (t >= total) return false;
  sample = t / tpf;
  const int p0 = (t - sample * tpf) * 64;
  if (lane >= min(64, a.hw_out - p0)) return false;
  const int q = p0 + lane;
  const int oh = q / a.w_out, ow = q - oh * a.w_out;
  ih0 = oh * a.s - 1;
  iw0 = ow * a.s - 1;
  return true;
}

template <int CO, typename TOut>
__device__ __forceinline__ void px3_store(const float (&acc)[CO], TOut* __restrict__ yp, int hw, int nco) {
  if (nco >= CO) {
#pragma unroll
    for (int co = 0; co < CO; ++co) yp[(int64_t)co * hw] = from_f32<TOut>(acc[co]);
  } else {
#pragma unroll
    for (int co = 0; co < CO; ++co)
      if (co < nco) yp[(int64_t)co * hw] = from_f32<TOut>(acc[co]);
  }
}

// H, spike and reset of one step with the membrane in acc: returns the
// spikes as one word (bit co = channel co0 + co fired).
template <int CO>
__device__ __forceinline__ uint32_t lif_fire(float (&acc)[CO], const LifCoef& L) {
  static_assert(CO <= 32, "one spike word per lane");
  uint32_t sw = 0u;
#pragma unroll
  for (int co = 0; co < CO; ++co) {
    const float h = L.decay_input ? acc[co] * L.inv_tau : acc[co];
    const bool fire = h >= L.v_th;
    sw |= (fire ? 1u : 0u) << co;
    acc[co] = L.hard ? (fire ? L.v_reset : h) : h - (fire ? L.v_th : 0.f);
  }
  return sw;
}

// One step's spikes of a tile (64 pixels from p0, npx of them present) to
// spk = the frame's plane of channel co0.
template <typename TOut, int CO>
__device__ __forceinline__ void px3_store_spikes(uint32_t sw, TOut* __restrict__ spk, int lane, int p0, int npx,
                                                 bool valid, bool mine, int nco, int hwo_t, int c_out_t) {
  if (nco == 32 && CO == 32 && (hwo_t & 3) == 0) {
    // Lane l stores pixels p0 + 4*(l & 15) .. +3 of channel 4*i + (l >> 4):
    // eight vector stores instead of 32 (npx is a multiple of 4).  The
    // lane-dependent offsets are formed here from a fresh opaque copy of
    // the lane index: hoisted out of the step loop they were spilled, and
    // the reload's wait for it (the vector memory counter retires in order)
    // also waited for the next step's prefetched bitmap words.
    int ls = lane;
    asm volatile("" : "+v"(ls));
    const int src = 4 * (ls & 15);
    uint32_t gw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) gw[j] = __shfl(sw, src + j);
    if (valid && src < npx) {
      constexpr int B = (int)sizeof(TOut);
      const auto sr = buf_rsrc(spk, (uint32_t)c_out_t * (uint32_t)hwo_t * B);
      const int cq = ls >> 4;
      const int vo = ((cq) * hwo_t + p0 + src) * B;
#pragma unroll
      for (int i = 0; i < CO / 4; ++i) {
        const int sh = 4 * i + cq;
        const uint32_t q = ((gw[0] >> sh) & 1u) | (((gw[1] >> sh) & 1u) << 1) | (((gw[2] >> sh) & 1u) << 2) |
                           (((gw[3] >> sh) & 1u) << 3);
        store_bits4<TOut>(q, sr, vo + 4 * i * hwo_t * B);
      }
    }
  } else if (mine) {
    for (int co = 0; co < nco; ++co)
      spk[(int64_t)co * hwo_t + p0 + lane] = from_f32<TOut>(((sw >> co) & 1u) ? 1.f : 0.f);
  }
}

// TOut is the spike type of the fused LIF kernel; the plain conv kernel
// takes its output type at run time (out_dtype) and ignores TOut.
template <typename TIn, typename TOut, int CO, bool LIF>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_px3(ConvArgs a, const uint32_t* __restrict__ bits,
                                                              const uint32_t* __restrict__ flags,
                                                              const TIn* __restrict__ x,
                                                              const float* __restrict__ wt,
                                                              const float* __restrict__ bias_p,
                                                              void* __restrict__ y, int groups, int nchunks,
                                                              int out_dtype) {
  typedef Px3Layout<CO> LY;
  extern __shared__ __align__(16) char smem[];
  const int lane0 = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // With 8 or more channel groups the default placement would give each XCD
  // one group over every frame, re-reading the whole bitmap through an L2
  // too small for it (layer4.0: 827 MB fetched for 61 MB of y + W); with
  // fewer groups the default placement measured faster.
  const int blk = groups >= 8 ? xcd_local_block((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int grp = blk % groups;
  const int co0 = grp * CO;
  const int krows = a.c_in * 9;
  const int hwo = a.hw_out;
  const int tpf = (hwo + 63) / 64;
  const int total = (int)a.n * tpf;   // LIF: a.n = samples, the T steps run inside a tile
  const int nblk = (int)(gridDim.x / groups);
  const bool resident = nchunks <= LY::resident_chunks;
  const int steps = LIF ? a.T : 1;
  const LifCoef L = lif_coef(a);
  // The group's bias (LIF: v_reset term + bias) in LDS: read per pass from
  // global memory it would be a vector load that waits for every store the
  // wavefront still has in flight.
  __shared__ float s_seed[CO];
  if (threadIdx.x < CO) {
    const int co = co0 + (int)threadIdx.x;
    const float b = (bias_p != nullptr && co < a.c_out) ? bias_p[co] : 0.f;
    s_seed[threadIdx.x] = LIF ? L.vr_term + b : b;
  }
  __syncthreads();

  if (resident) {
    for (int c = 0; c < nchunks; ++c)
      load_chunk_px3<CO>(smem + c * LY::chunk_bytes, wt, c, krows, a.c_out, co0, wave, lane0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // First-chunk bitmap words of the next tile (or the next step) are always
  // requested before the current tile's (step's) stores: the vector memory
  // counter retires in issue order, so words requested after the 64 stores
  // of a tile would make their first use wait for all of those stores.
  uint32_t wn[9];
  if constexpr (!LIF) {
    int ih0, iw0, sample;
    if (px3_tile(a, (blk / groups) * kRowsWaves + wave, lane0, total, tpf, sample, ih0, iw0))
      px3_load_words(wn, bits + (int64_t)sample * a.hw_in * a.cwp, a, ih0, iw0, 0);
  }
  // Passes of kRowsWaves tiles.  With streamed chunks every wavefront takes
  // part in every barrier, including those of a pass past the end.
  for (int pass = blk / groups; pass * kRowsWaves < total; pass += nblk) {
    // Lane-dependent addresses are recomputed in every pass rather than kept
    // live across the loop (the accumulators need the registers).
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int t = pass * kRowsWaves + wave;
    const bool valid = t < total;
    const int sample = valid ? t / tpf : 0;
    const int p0 = valid ? (t - sample * tpf) * 64 : 0;
    const int npx = min(64, hwo - p0);
    const bool mine = valid && lane < npx;
    // This lane's output pixel and the top-left corner of its input window.
    const int q = p0 + min(lane, npx - 1);
    const int oh = q / a.w_out, ow = q - (q / a.w_out) * a.w_out;
    const int ih0 = oh * a.s - 1, iw0 = ow * a.s - 1;
    // Per-channel values (bias, store offsets) are formed in every pass,
    // not kept live across the loop: the accumulators need the registers.
    int hwo_t = hwo, c_out_t = a.c_out;
    asm volatile("" : "+s"(hwo_t), "+s"(c_out_t));
    const int nco = min(CO, c_out_t - co0);
    float acc[CO];
    if constexpr (LIF) {
      // Membrane before step 0: v_init or 0.
      const float* vi = a.v_init;
#pragma unroll
      for (int co = 0; co < CO; ++co) acc[co] = 0.f;
      if (vi != nullptr && mine) {
        const float* vp = vi + ((int64_t)sample * c_out_t + co0) * hwo_t + p0 + lane;
#pragma unroll
        for (int co = 0; co < CO; ++co)
          if (co < nco) acc[co] = vp[(int64_t)co * hwo_t];
      }
    } else {
#pragma unroll
      for (int co = 0; co < CO; ++co) acc[co] = s_seed[co];
    }
    // The fused LIF kernel requests a tile's first words here; it prefetches
    // per step instead (the T steps of a tile are its long stretch of work).
    if constexpr (LIF)
      if (mine) px3_load_words(wn, bits + (int64_t)sample * a.hw_in * a.cwp, a, ih0, iw0, 0);
    for (int st = 0; st < steps; ++st) {
      const int64_t frame = LIF ? (int64_t)st * a.n + sample : sample;
      if constexpr (LIF) lif_seed_lds<CO>(acc, L, s_seed);
      bool value = false;
      if (valid) {
        const int oh_a = p0 / a.w_out, oh_b = (p0 + npx - 1) / a.w_out;
        value = rows_value_path(a, flags, frame, oh_a * a.s - 1, oh_b * a.s + 1);
      }
      const uint32_t* __restrict__ bf = bits + frame * a.hw_in * a.cwp;
      const TIn* __restrict__ xf = x + frame * a.c_in * a.hw_in;
      if (!resident) {
        __syncthreads();  // the previous step/pass is done with both buffers
        // The streaming addresses are formed here, not hoisted to the pass
        // start: kept live they would be spilled to scratch on every pass,
        // resident or not.
        int ll = lane;
        asm volatile("" : "+v"(ll));
        load_chunk_px3<CO>(smem, wt, 0, krows, a.c_out, co0, wave, ll);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
      for (int c = 0; c < nchunks; ++c) {
        // Stream chunk c+1 into the other buffer; it was last read during
        // chunk c-1, which every wavefront finished before the last barrier.
        if (!resident && c + 1 < nchunks) {
          int ll = lane;
          asm volatile("" : "+v"(ll));
          load_chunk_px3<CO>(smem + ((c + 1) & 1) * LY::chunk_bytes, wt, c + 1, krows, a.c_out, co0, wave, ll);
        }
        if (mine) {
          // This chunk's words were loaded during the previous chunk's walk;
          // start the next chunk's loads now.
          uint32_t w[9];
#pragma unroll
          for (int tp = 0; tp < 9; ++tp) w[tp] = wn[tp];
          // Opaque to the optimiser: a select between two array elements
          // would otherwise be folded into an indexed load, which keeps the
          // array in scratch memory.
          asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]),
                       "+v"(w[7]), "+v"(w[8]));
          if (c + 1 < nchunks) px3_load_words(wn, bf, a, ih0, iw0, c + 1);
          uint32_t nz = 0u;
#pragma unroll
          for (int tp = 0; tp < 9; ++tp) nz |= (w[tp] != 0u ? 1u : 0u) << tp;
          const char* chunk = smem + (resident ? c : (c & 1)) * LY::chunk_bytes;
          uint32_t m = 0u;
          int tap = 0;
          // Per-lane cursor over (tap, ci): the wavefront loops while any
          // lane has spikes left.
          while ((m | nz) != 0u) {
            if (m == 0u) {
              tap = __builtin_ctz(nz);
              nz &= nz - 1u;
              m = px3_select(w, tap);
            }
            const int bit = __builtin_ctz(m);
            m &= m - 1u;
            float xv = 1.f;
            if (value) {
              const int ih = ih0 + tap / 3, iw = iw0 + tap % 3;
              xv = to_f32<TIn>(xf[(int64_t)(c * kPx3Ch + bit) * a.hw_in + ih * a.w_in + iw]);
              // Waited for here, in the value path: otherwise every round's
              // products wait for all memory operations in flight, which
              // include the next chunk's streamed rows and bitmap words.
              __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
            }
            px3_add_row<CO, !LIF>(acc, chunk, bit * 9 + tap, xv);
          }
        }
        if (!resident) {
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
        }
      }
      if constexpr (LIF) {
        // H, spike and the reset: the spikes are collected as one word per
        // 32 channels (the membrane stays in acc), the next step's words are
        // requested, then the spikes are stored.
        const uint32_t sw = lif_fire<CO>(acc, L);
        if (st + 1 < steps && mine)
          px3_load_words(wn, bits + (frame + a.n) * a.hw_in * a.cwp, a, ih0, iw0, 0);
        __builtin_amdgcn_sched_barrier(0);
        TOut* __restrict__ spk = static_cast<TOut*>(y) + (frame * c_out_t + co0) * hwo_t;
        px3_store_spikes<TOut, CO>(sw, spk, lane, p0, npx, valid, mine, nco, hwo_t, c_out_t);
      }
    }
    if constexpr (!LIF) {
      int nih0, niw0, nsample;
      if (px3_tile(a, (pass + nblk) * kRowsWaves + wave, lane, total, tpf, nsample, nih0, niw0))
        px3_load_words(wn, bits + (int64_t)nsample * a.hw_in * a.cwp, a, nih0, niw0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (mine) {
      if constexpr (LIF) {
        const int64_t vb = ((int64_t)sample * c_out_t + co0) * hwo_t + p0 + lane;
        px3_store<CO>(acc, a.v_out + vb, hwo_t, nco);
      } else {
        const int64_t yb = ((int64_t)sample * c_out_t + co0) * hwo_t + p0 + lane;
        if (out_dtype == SF_F16) px3_store<CO>(acc, static_cast<__half*>(y) + yb, hwo_t, nco);
        else if (out_dtype == SF_BF16) px3_store<CO>(acc, static_cast<__hip_bfloat16*>(y) + yb, hwo_t, nco);
        else px3_store<CO>(acc, static_cast<float*>(y) + yb, hwo_t, nco);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streamed variant for C_in > 128 (64 output channels per workgroup, weight
// chunks of 32 input channels streamed through the two LDS buffers) over
// tiles of the flattened (frame, pixel) axis: all 64 lanes carry an output
// pixel on planes of 49 or 196 pixels (per-frame tiles leave 23% of them
// idle there), and the host sizes the workgroup so that the wave-tiles
// spread evenly over the CUs (one workgroup per CU, since the two chunk
// buffers fill the LDS).  A lane's frame, input window and output offsets
// are its own; the walk and the chunk pipeline are k_conv_px3's.  Output
// element (co, oh, ow) = bias[co] + its active taps summed by one lane in
// (chunk, tap, ci) order, as there.
// ---------------------------------------------------------------------------

// Direct-to-LDS loads of chunk c by the nw wavefronts of the workgroup.
__device__ __forceinline__ void load_chunk_px3_nw(char* buf, const float* __restrict__ wt, int c, int krows,
                                                  int c_out, int co0, int wave, int nw, int lane) {
  typedef Px3Layout<64> L;
  for (int u = wave; u < L::units; u += nw) {
    const int pos = u * 64 + lane;
    const int r = pos / L::stride;
    const int q = pos - r * L::stride;
    const int row = c * kPx3Rows + r;
    const int col = co0 + 4 * q;
    const float* src = (q < L::pieces && r < kPx3Rows && row < krows && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
  }
}

// dq (nullable): the dense-tile queue.  A binary wave-tile with a pixel of
// kDenseLaneSpikes or more spikes in the first chunk is appended to its
// group's queue and neither walked nor stored here: the matrix-core kernel
// launched next computes it (sf_dense_mfma.hip).
template <typename TIn, typename TOut>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_px3s(ConvArgs a, const uint32_t* __restrict__ bits,
                                                               const uint32_t* __restrict__ flags,
                                                               const TIn* __restrict__ x, const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p, TOut* __restrict__ y,
                                                               int groups, int nchunks, DenseQueue* __restrict__ dq) {
  typedef Px3Layout<64> LY;
  extern __shared__ __align__(16) char smem[];
  __shared__ float s_seed[64];
  const int nw = __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = groups >= 8 ? xcd_local_block((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const int krows = a.c_in * 9;
  const int hwo = a.hw_out;
  const int total_px = (int)(a.n * hwo);  // below 2^31 (the host checks the output size)
  const int total = (total_px + 63) / 64;
  const int nblk = (int)(gridDim.x / groups);
  const uint32_t frame_bytes = (uint32_t)a.hw_in * (uint32_t)a.cwp * 4u;
  const auto rs_bits = buf_rsrc(bits, (uint32_t)((int64_t)a.n * frame_bytes));
  if (threadIdx.x < 64) {
    const int co = co0 + (int)threadIdx.x;
    s_seed[threadIdx.x] = (bias_p != nullptr && co < a.c_out) ? bias_p[co] : 0.f;
  }
  for (int pass = blk / groups; pass * nw < total; pass += nblk) {
    // The lane index is formed anew in each pass (in asm, which the
    // optimiser cannot hoist): kept live across the loop it was spilled, and
    // its reload waited for the previous pass's stores.
    int lane;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
    const int t = pass * nw + wave;
    const int g = t * 64 + lane;
    const bool mine = g < total_px;
    const int gc = mine ? g : total_px - 1;  // lanes past the end form valid addresses
    const int sample = gc / hwo;
    const int q = gc - sample * hwo;
    const int oh = q / a.w_out, ow = q - (q / a.w_out) * a.w_out;
    const int ih0 = oh * a.s - 1, iw0 = ow * a.s - 1;
    const uint32_t fbase = (uint32_t)sample * frame_bytes;
    // The lane's output offset (bytes), formed here so that only it, not the
    // pixel index, stays live across the chunk loop; lanes without a pixel
    // start past the end of y.
    constexpr uint32_t B = (uint32_t)sizeof(TOut);
    const uint32_t yrange = (uint32_t)total_px * (uint32_t)a.c_out * B;
    uint32_t ybase =
        mine ? (((uint32_t)sample * (uint32_t)a.c_out + (uint32_t)co0) * (uint32_t)hwo + (uint32_t)q) * B : yrange;
    // This pass's first words, in flight during the first chunk's load.
    uint32_t wn[9];
    px3_load_words_at(wn, rs_bits, fbase, a, ih0, iw0, 0);
    // The multiply-by-x path for the whole tile when any lane's input rows
    // hold a non-binary value.
    const bool value = __ballot(mine && rows_value_path(a, flags, sample, ih0, ih0 + 2)) != 0ull;
    // Dense-tile branch: a binary wave-tile whose first chunk is dense is
    // queued for the matrix cores instead of walked (its lanes then store
    // nothing here).
    bool walk = mine;
    if (dq != nullptr && !value) {
      uint32_t cnt = 0u;
#pragma unroll
      for (int tp = 0; tp < 9; ++tp) cnt += (uint32_t)__popc(wn[tp]);
      if (__ballot(mine && cnt >= (uint32_t)kDenseLaneSpikes) != 0ull) {
        uint32_t slot = 0u;
        if (lane == 0) slot = atomicAdd(&dq->count[grp], 1u);
        slot = __builtin_amdgcn_readfirstlane(slot);
        if (slot < (uint32_t)kDenseQueueCap) {
          if (lane == 0) {
            dq->start[grp][slot] = (uint32_t)t * 64u;
            dq->npx[grp][slot] = 64;  // the last tile's pixels past the end are not stored
          }
          walk = false;
          ybase = yrange;
        }
      }
    }
    __syncthreads();  // the previous pass is done with both buffers (and s_seed is written)
    {
      int ll = lane;
      asm volatile("" : "+v"(ll));
      load_chunk_px3_nw(smem, wt, 0, krows, a.c_out, co0, wave, nw, ll);
    }
    float acc[64];
#pragma unroll
    for (int co = 0; co < 64; ++co) acc[co] = s_seed[co];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
      // Chunk c+1 streams into the other buffer; it was last read during
      // chunk c-1, which every wavefront finished before the last barrier.
      if (c + 1 < nchunks) {
        int ll = lane;
        asm volatile("" : "+v"(ll));
        load_chunk_px3_nw(smem + ((c + 1) & 1) * LY::chunk_bytes, wt, c + 1, krows, a.c_out, co0, wave, nw, ll);
      }
      uint32_t w[9];
#pragma unroll
      for (int tp = 0; tp < 9; ++tp) w[tp] = wn[tp];
      // Opaque to the optimiser: a select between array elements would
      // otherwise be folded into an indexed load from scratch memory.
      asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]),
                   "+v"(w[7]), "+v"(w[8]));
      if (c + 1 < nchunks) px3_load_words_at(wn, rs_bits, fbase, a, ih0, iw0, c + 1);
      if (walk) {
        uint32_t nz = 0u;
#pragma unroll
        for (int tp = 0; tp < 9; ++tp) nz |= (w[tp] != 0u ? 1u : 0u) << tp;
        const char* chunk = smem + (c & 1) * LY::chunk_bytes;
        uint32_t m = 0u;
        const char* trows = chunk;
        // Per-lane cursor over (tap, ci): the wavefront loops while any
        // lane has spikes left.
        while ((m | nz) != 0u) {
          if (m == 0u) {
            const int tap = __builtin_ctz(nz);
            nz &= nz - 1u;
            m = px3_select(w, tap);
            trows = px3_tap_rows(chunk, tap);
          }
          const int bit = __builtin_ctz(m);
          m &= m - 1u;
          float xv = 1.f;
          if (value) {
            const int tap = px3_rows_tap(chunk, trows);
            const int ih = ih0 + tap / 3, iw = iw0 + tap % 3;
            const TIn* __restrict__ xf = x + (int64_t)sample * a.c_in * a.hw_in;
            xv = to_f32<TIn>(xf[(int64_t)(c * kPx3Ch + bit) * a.hw_in + ih * a.w_in + iw]);
            // Waited for here, in the value path: otherwise every round's
            // products wait for the next chunk's rows and words too.
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
          }
          px3_add_row_at<64>(acc, px3_spike_row(trows, bit), 0, xv);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    {
      // Every frame's output planes as one buffer (below 2^31 bytes): lanes
      // without a pixel start at its end; channels past C_out are skipped.
      int hwo_t = hwo, c_out_t = a.c_out;
      asm volatile("" : "+s"(hwo_t), "+s"(c_out_t));
      const int nco = min(64, c_out_t - co0);
      const auto rs = buf_rsrc(y, yrange);
      const uint32_t plane = (uint32_t)hwo_t * B;
      uint32_t off = ybase;
#pragma unroll
      for (int co = 0; co < 64; ++co) {
        if (co < nco) BufIO<TOut>::store(from_f32<TOut>(acc[co]), rs, (int)off, 0);
        off += plane;
        asm volatile("" : "+v"(off));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide-chunk variant of the plain conv for C_in <= 64 and 64 output channels
// per workgroup: the weight rows of all 64 input channels (576 rows of 272
// bytes, 156.7 KB) are resident, and each lane walks its nine taps'
// 64-channel words in one pass instead of two 32-channel chunks.  A tile's
// round count is its busiest pixel's spike count; over 64 channels at once
// it is ~19% below the sum over two 32-channel chunks (the maximum over a
// tile's lanes grows more slowly than the mean).  Output element (co, oh,
// ow) = bias[co] + its active taps summed by one lane in (tap, ci) order.
// ---------------------------------------------------------------------------
constexpr int kPx3wRows = 64 * 9;
constexpr int kPx3wUnits = (kPx3wRows * 17 + 63) / 64;  // 1 KB load units
constexpr int kPx3wBytes = kPx3wUnits * 1024;           // 156,672
// 32 output channels: the rows of up to 128 input channels (1152 rows of
// 128 bytes, the 32-channel slice layout of Px3Layout<32>).
constexpr int kPx3w32Rows = 128 * 9;
constexpr int kPx3w32Units = kPx3w32Rows * 8 / 64;      // 1 KB load units
constexpr int kPx3w32Bytes = kPx3w32Units * 1024;       // 147,456

template <int CO>
constexpr int px3w_bytes() { return CO == 64 ? kPx3wBytes : kPx3w32Bytes; }

// Direct-to-LDS loads of the resident rows.  CO = 64: 576 rows padded to 17
// pieces of 16 bytes; CO = 32: up to 1152 rows of 8 pieces, piece s of row r
// stored at position s ^ ((r >> 1) & 7) (Px3Layout<32>; the swizzle key of a
// row is the same whether it is indexed within its 32-channel chunk or across
// the chunks, 288 rows being a multiple of 16).  Pads, rows past C_in and
// channels past C_out read a valid but unrelated address whose values are
// never used.
template <int CO>
__device__ __forceinline__ void load_rows_px3w(char* buf, const float* __restrict__ wt, int krows, int c_out, int co0,
                                               int wave, int nw, int lane) {
  if constexpr (CO == 64) {
    for (int u = wave; u < kPx3wUnits; u += nw) {
      const int pos = u * 64 + lane;
      const int r = pos / 17, q = pos - r * 17;
      const int col = co0 + 4 * q;
      const float* src = (q < 16 && r < krows && col < c_out) ? wt + (int64_t)r * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  } else {
    for (int u = wave; u < kPx3w32Units; u += nw) {
      const int pos = u * 64 + lane;
      const int r = pos >> 3, q = pos & 7;
      const int col = co0 + 4 * (q ^ ((r >> 1) & 7));
      const float* src = (r < krows && col < c_out) ? wt + (int64_t)r * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  }
}

// Channel words c0 and c0 + 1 (a 64-channel super-chunk) of the lane's nine
// taps (0 outside the frame; the second is 0 past the pixel's last word),
// bf = the frame's bitmap, through one buffer resource as in px3_load_words.
__device__ __forceinline__ void px3w_load_words(uint32_t (&lo)[9], uint32_t (&hi)[9], const uint32_t* __restrict__ bf,
                                                const ConvArgs& a, int ih0, int iw0, int c0) {
  const uint32_t frame_bytes = (uint32_t)a.hw_in * (uint32_t)a.cwp * 4u;
  const auto rs = buf_rsrc(bf, frame_bytes);
  const bool two = c0 + 1 < a.cwp;
  const uint32_t cofs = (uint32_t)c0 * (uint32_t)a.bm_ws;
  const uint32_t next = (uint32_t)a.bm_ws * 4u;  // bytes from word c0 to word c0 + 1 of a pixel
#pragma unroll
  for (int tp = 0; tp < 9; ++tp) {
    const int ih = ih0 + tp / 3, iw = iw0 + tp % 3;
    const bool in = ih >= 0 && ih < a.h_in && iw >= 0 && iw < a.w_in;
    const uint32_t off = in ? ((uint32_t)(ih * a.w_in + iw) * (uint32_t)a.bm_ps + cofs) * 4u : 0x80000000u;
    lo[tp] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0);
    // The whole offset in the VGPR (soffset stays 0, as in every buffer
    // access of this library); past the frame it stays past num_records.
    hi[tp] = two ? __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(off + next), 0, 0) : 0u;
  }
}

// Stores and waits: a tile's channel stores are issued unconditionally
// (buffer stores; pixels past the tile and channels past C_out fall outside
// the buffer's range and are dropped), and the bitmap walk has no memory
// loads of its own, so the compiler can count exactly how many stores
// follow the next tile's word loads: the walk then waits for those loads
// only, not for the previous tile's stores.  (With conditional stores the
// count differed between paths and the merged wait drained nearly all of
// them before every walk.)
//
// CO = 32 (64 < C_in <= 128): the same walk over up to two 64-channel
// super-chunks, the second's words requested before the first's walk; rows
// (64 sc + ci) * 9 + tap of the resident 32-channel slice layout.
//
// LIF (CO = 32): the fused conv-LIF of k_conv_px3<LIF> on this walk: the
// membrane stays in acc over the T steps of a tile, each step's spikes are
// stored as 4-pixel vectors after the next step's first words are
// requested, and v_T is stored at the end; y is then the spike tensor.
template <typename TIn, typename TOut, int CO, bool LIF>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_px3w(ConvArgs a, const uint32_t* __restrict__ bits,
                                                               const uint32_t* __restrict__ flags,
                                                               const TIn* __restrict__ x, const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p, TOut* __restrict__ y,
                                                               int groups) {
  static_assert(!LIF || CO == 32, "the fused LIF form keeps one spike word per lane");
  extern __shared__ __align__(16) char smem[];
  __shared__ float s_seed[CO];
  const int lane0 = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6));  // tiles per pass
  const int blk = groups >= 8 ? xcd_local_block((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int grp = blk % groups;
  const int co0 = grp * CO;
  const int hwo = a.hw_out;
  const int tpf = (hwo + 63) / 64;
  const int total = (int)a.n * tpf;  // LIF: a.n = samples, the T steps run inside a tile
  const int nblk = (int)(gridDim.x / groups);
  const int nsc = CO == 64 ? 1 : (a.cwp + 1) / 2;  // 64-channel super-chunks
  const int steps = LIF ? a.T : 1;
  const LifCoef L = lif_coef(a);
  if (threadIdx.x < CO) {
    const int co = co0 + (int)threadIdx.x;
    const float b = (bias_p != nullptr && co < a.c_out) ? bias_p[co] : 0.f;
    s_seed[threadIdx.x] = LIF ? L.vr_term + b : b;
  }
  load_rows_px3w<CO>(smem, wt, a.c_in * 9, a.c_out, co0, wave, nw, lane0);
  // The first tile's words; later tiles' are requested before the previous
  // tile's stores (the vector memory counter retires in issue order).  The
  // fused LIF form requests a tile's first words at the tile and prefetches
  // per step (the T steps of a tile are its long stretch of work).
  uint32_t nlo[9], nhi[9];
  if constexpr (!LIF) {
    const int t = (blk / groups) * nw + wave;
    if (t < total) {
      const int sample = t / tpf, p0 = (t - sample * tpf) * 64;
      const int q = p0 + min(lane0, hwo - p0 - 1);
      const int oh = q / a.w_out, ow = q - oh * a.w_out;
      px3w_load_words(nlo, nhi, bits + (int64_t)sample * a.hw_in * a.cwp, a, oh * a.s - 1, ow * a.s - 1, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's direct weight loads have landed
  __syncthreads();
  for (int pass = blk / groups; pass * nw < total; pass += nblk) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int t = pass * nw + wave;
    const bool valid = t < total;
    const int sample = valid ? t / tpf : 0;
    const int p0 = valid ? (t - sample * tpf) * 64 : 0;
    const int npx = min(64, hwo - p0);
    const bool mine = valid && lane < npx;
    const int q = p0 + min(lane, npx - 1);
    const int oh = q / a.w_out, ow = q - (q / a.w_out) * a.w_out;
    const int ih0 = oh * a.s - 1, iw0 = ow * a.s - 1;
    int hwo_t = hwo, c_out_t = a.c_out;
    asm volatile("" : "+s"(hwo_t), "+s"(c_out_t));
    float acc[CO];
    if constexpr (LIF) {
      // Membrane before step 0: v_init or 0.
      const int nco = min(CO, c_out_t - co0);
      const float* vi = a.v_init;
#pragma unroll
      for (int co = 0; co < CO; ++co) acc[co] = 0.f;
      if (vi != nullptr && mine) {
        const float* vp = vi + ((int64_t)sample * c_out_t + co0) * hwo_t + p0 + lane;
#pragma unroll
        for (int co = 0; co < CO; ++co)
          if (co < nco) acc[co] = vp[(int64_t)co * hwo_t];
      }
      px3w_load_words(nlo, nhi, bits + (int64_t)sample * a.hw_in * a.cwp, a, ih0, iw0, 0);
    } else {
#pragma unroll
      for (int co = 0; co < CO; ++co) acc[co] = s_seed[co];
    }
    for (int st = 0; st < steps; ++st) {
      const int64_t frame = LIF ? (int64_t)st * a.n + sample : sample;
      if constexpr (LIF) lif_seed_lds<CO>(acc, L, s_seed);
      bool value = false;
      if (valid) {
        const int oh_a = p0 / a.w_out, oh_b = (p0 + npx - 1) / a.w_out;
        value = rows_value_path(a, flags, frame, oh_a * a.s - 1, oh_b * a.s + 1);
      }
      const uint32_t* __restrict__ bf = bits + frame * a.hw_in * a.cwp;
      const TIn* __restrict__ xf = x + frame * a.c_in * a.hw_in;
      for (int sc = 0; sc < nsc; ++sc) {
        uint32_t wl[9], wh[9];
#pragma unroll
        for (int tp = 0; tp < 9; ++tp) {
          wl[tp] = nlo[tp];
          wh[tp] = nhi[tp];
        }
        // Opaque to the optimiser: a select between array elements would
        // otherwise be folded into an indexed load from scratch memory.
        asm volatile("" : "+v"(wl[0]), "+v"(wl[1]), "+v"(wl[2]), "+v"(wl[3]), "+v"(wl[4]), "+v"(wl[5]), "+v"(wl[6]),
                     "+v"(wl[7]), "+v"(wl[8]));
        asm volatile("" : "+v"(wh[0]), "+v"(wh[1]), "+v"(wh[2]), "+v"(wh[3]), "+v"(wh[4]), "+v"(wh[5]), "+v"(wh[6]),
                     "+v"(wh[7]), "+v"(wh[8]));
        // The next super-chunk's words are in flight during this walk.
        if (CO != 64 && sc + 1 < nsc) px3w_load_words(nlo, nhi, bf, a, ih0, iw0, 2 * (sc + 1));
        if (mine) {
          uint32_t nz = 0u;
#pragma unroll
          for (int tp = 0; tp < 9; ++tp) nz |= ((wl[tp] | wh[tp]) != 0u ? 1u : 0u) << tp;
          const int row0 = 64 * sc * 9;
          // Per-lane cursor over (tap, ci): the wavefront loops while any
          // lane has spikes left.
          uint64_t m = 0ull;
          int tap = 0;               // CO = 32
          const char* trows = smem;  // CO = 64: the tap's rows (row0 = 0)
          while ((m != 0ull) || (nz != 0u)) {
            if (m == 0ull) {
              const int t = __builtin_ctz(nz);
              nz &= nz - 1u;
              m = ((uint64_t)px3_select(wh, t) << 32) | px3_select(wl, t);
              if constexpr (CO == 64) trows = px3_tap_rows(smem, t);
              else tap = t;
            }
            const int bit = __builtin_ctzll(m);
            m &= m - 1ull;
            float xv = 1.f;
            if (value) {
              int ih = ih0, iw = iw0;
              if constexpr (CO == 64) {
                // The tap and the lane's window origin formed here (the
                // lane index anew, in asm): kept live across the walk they
                // take registers the walk needs.
                tap = px3_rows_tap(smem, trows);
                int ln;
                asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
                const int qv = p0 + min(ln, npx - 1);
                const int ohv = qv / a.w_out;
                ih = ohv * a.s - 1;
                iw = (qv - ohv * a.w_out) * a.s - 1;
              }
              ih += tap / 3;
              iw += tap % 3;
              xv = to_f32<TIn>(xf[(int64_t)(64 * sc + bit) * a.hw_in + ih * a.w_in + iw]);
              // Waited for here, in the value path: otherwise the products
              // below wait for every memory operation in flight (the
              // previous tile's stores included) on every spike of the
              // bitmap path too.
              __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
            }
            if constexpr (CO == 64) px3_add_row_at<64>(acc, px3_spike_row(trows, bit), 0, xv);
            else px3_add_row<CO, !LIF>(acc, smem, row0 + bit * 9 + tap, xv);
          }
        }
      }
      if constexpr (LIF) {
        // Spikes and reset; the next step's first words are requested
        // before the spike stores.
        const int nco = min(CO, c_out_t - co0);
        const uint32_t sw = lif_fire<CO>(acc, L);
        if (st + 1 < steps)
          px3w_load_words(nlo, nhi, bits + (frame + a.n) * a.hw_in * a.cwp, a, ih0, iw0, 0);
        __builtin_amdgcn_sched_barrier(0);
        TOut* __restrict__ spk = y + (frame * c_out_t + co0) * hwo_t;
        px3_store_spikes<TOut, CO>(sw, spk, lane, p0, npx, valid, mine, nco, hwo_t, c_out_t);
      }
    }
    if constexpr (LIF) {
      if (mine) {
        const int64_t vb = ((int64_t)sample * c_out_t + co0) * hwo_t + p0 + lane;
        px3_store<CO>(acc, a.v_out + vb, hwo_t, min(CO, c_out_t - co0));
      }
    } else {
      {
        const int tn = (pass + nblk) * nw + wave;
        if (tn < total) {
          const int ns = tn / tpf, np0 = (tn - ns * tpf) * 64;
          const int nq = np0 + min(lane, hwo - np0 - 1);
          const int noh = nq / a.w_out, now = nq - noh * a.w_out;
          px3w_load_words(nlo, nhi, bits + (int64_t)ns * a.hw_in * a.cwp, a, noh * a.s - 1, now * a.s - 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // The sample's output planes as one buffer: lanes without a pixel
      // start at its end, channels past C_out land past it too (the host
      // keeps (C_out + CO) planes below 2^31 bytes, so no offset wraps).
      constexpr uint32_t B = (uint32_t)sizeof(TOut);
      const uint32_t range = (uint32_t)c_out_t * (uint32_t)hwo_t * B;
      const auto rs = buf_rsrc(y + (int64_t)sample * c_out_t * hwo_t, range);
      const uint32_t base = mine ? ((uint32_t)co0 * (uint32_t)hwo_t + (uint32_t)(p0 + lane)) * B : range;
      const uint32_t plane = (uint32_t)hwo_t * B;
      // One offset register stepped by a plane per store (opaque, so the
      // offsets are not precomputed into registers); soffset stays 0.
      // Planes of whole 128-byte lines (tiles then start on a line) are
      // streamed out.
      uint32_t off = base;
      if ((plane & 127u) == 0u) {
#pragma unroll
        for (int co = 0; co < CO; ++co) {
          BufIO<TOut>::template store<kStoreStream>(from_f32<TOut>(acc[co]), rs, (int)off, 0);
          off += plane;
          asm volatile("" : "+v"(off));
        }
      } else {
#pragma unroll
        for (int co = 0; co < CO; ++co) {
          BufIO<TOut>::store(from_f32<TOut>(acc[co]), rs, (int)off, 0);
          off += plane;
          asm volatile("" : "+v"(off));
        }
      }
    }
  }
}

template <typename TIn, typename TOut, int CO, bool LIF = false>
int launch_px3w_to(const ConvArgs& a, hipStream_t stream) {
  const int groups = (a.c_out + CO - 1) / CO;
  const int64_t tiles = a.n * (int64_t)((a.hw_out + 63) / 64);
  // One workgroup per CU (the weights fill the LDS) making the same number
  // of passes: as many as 16-wave workgroups would need, with the wave-tiles
  // spread evenly over them (no CU idles through another's last pass).
  const int nw = even_pass_waves(tiles * groups);
  const int64_t passes = (tiles * groups + (int64_t)num_cus() * nw - 1) / ((int64_t)num_cus() * nw);
  const int64_t per_group = (tiles + (int64_t)nw * passes - 1) / ((int64_t)nw * passes);
  const int grid = (int)(groups * (per_group > 0 ? per_group : 1));
  constexpr auto kern = k_conv_px3w<TIn, TOut, CO, LIF>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes - 1024);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), (size_t)px3w_bytes<CO>(), stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, static_cast<TOut*>(a.y), groups);
  return (int)hipGetLastError();
}

template <typename TIn, int CO>
int launch_px3w_t(const ConvArgs& a, int out_dtype, hipStream_t stream) {
  if (out_dtype == SF_F16) return launch_px3w_to<TIn, __half, CO>(a, stream);
  if (out_dtype == SF_BF16) return launch_px3w_to<TIn, __hip_bfloat16, CO>(a, stream);
  return launch_px3w_to<TIn, float, CO>(a, stream);
}

template <typename TIn, typename TOut, int CO, bool LIF>
int launch_px3_t(const ConvArgs& a, int out_dtype, hipStream_t stream) {
  typedef Px3Layout<CO> LY;
  const int groups = (a.c_out + CO - 1) / CO;
  const int nchunks = (a.c_in + kPx3Ch - 1) / kPx3Ch;
  const int held = nchunks <= LY::resident_chunks ? nchunks : 2;
  const size_t lds = (size_t)held * LY::chunk_bytes;
  const int64_t tiles = a.n * (int64_t)((a.hw_out + 63) / 64);
  const int64_t need = (tiles + kRowsWaves - 1) / kRowsWaves;
  const int per_group = (int)(need < num_cus() ? need : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_px3<TIn, TOut, CO, LIF>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes - 1024);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kRowsWaves), lds, stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, a.y, groups, nchunks, out_dtype);
  return (int)hipGetLastError();
}

template <typename TIn, typename TOut>
int launch_px3s_to(const ConvArgs& a, hipStream_t stream, DenseQueue** dense) {
  typedef Px3Layout<64> LY;
  const int groups = (a.c_out + 63) / 64;
  const int nchunks = (a.c_in + kPx3Ch - 1) / kPx3Ch;
  const int64_t tiles = (a.n * (int64_t)a.hw_out + 63) / 64;
  const int nw = even_pass_waves(tiles * groups);
  const int64_t per_group = (tiles + nw - 1) / nw;
  const int grid = (int)(groups * per_group);
  constexpr auto kern = k_conv_px3s<TIn, TOut>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes - 1024);
  if (e != (int)hipSuccess) return e;
  // (Queue entries hold a run's first pixel of the flattened axis in 31 bits.)
  DenseQueue* dq =
      groups <= kDenseQueueGroups && a.n * (int64_t)a.hw_out < (1ll << 31) ? dense_queue_for(stream) : nullptr;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), (size_t)2 * LY::chunk_bytes, stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, static_cast<TOut*>(a.y), groups, nchunks, dq);
  const int rc = (int)hipGetLastError();
  if (rc == (int)hipSuccess) *dense = dq;
  return rc;
}

template <typename TIn>
int launch_px3s_t(const ConvArgs& a, int out_dtype, hipStream_t stream, DenseQueue** dense) {
  if (out_dtype == SF_F16) return launch_px3s_to<TIn, __half>(a, stream, dense);
  if (out_dtype == SF_BF16) return launch_px3s_to<TIn, __hip_bfloat16>(a, stream, dense);
  return launch_px3s_to<TIn, float>(a, stream, dense);
}

template <int CO>
int launch_px3_co(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  if (in_dtype == SF_F16) return launch_px3_t<__half, float, CO, false>(a, out_dtype, stream);
  if (in_dtype == SF_BF16) return launch_px3_t<__hip_bfloat16, float, CO, false>(a, out_dtype, stream);
  return launch_px3_t<float, float, CO, false>(a, out_dtype, stream);
}

// Output channels per workgroup slice: 64, or 32 where that keeps the
// weights resident in LDS (64 < C_in <= 128), which removes the per-pass
// chunk streaming and its barriers at the cost of walking the spikes once
// per slice.  (A 16-channel slice, resident up to C_in = 256, walks too
// often: slower than streaming.)
int launch_px3_conv(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream, DenseQueue** dense) {
  // C_in <= 64: one 64-channel super-chunk, every weight row resident, 64
  // output channels; 64 < C_in <= 128: 32-channel slices of all 128 input
  // channels' rows, two super-chunks.  (One sample's output planes must be
  // addressable by one buffer resource, with CO planes to spare.)
  const int out_bytes = out_dtype == SF_F32 ? 4 : 2;
  if ((int64_t)(a.c_out + 64) * a.hw_out * out_bytes < 0x7fffffffLL) {
    if (a.c_in <= 64 && a.cwp <= 2) {
      if (in_dtype == SF_F16) return launch_px3w_t<__half, 64>(a, out_dtype, stream);
      if (in_dtype == SF_BF16) return launch_px3w_t<__hip_bfloat16, 64>(a, out_dtype, stream);
      return launch_px3w_t<float, 64>(a, out_dtype, stream);
    }
    if (a.c_in <= 128 && a.cwp <= 4) {
      if (in_dtype == SF_F16) return launch_px3w_t<__half, 32>(a, out_dtype, stream);
      if (in_dtype == SF_BF16) return launch_px3w_t<__hip_bfloat16, 32>(a, out_dtype, stream);
      return launch_px3w_t<float, 32>(a, out_dtype, stream);
    }
  }
  const int nch = (a.c_in + kPx3Ch - 1) / kPx3Ch;
  if (nch > Px3Layout<64>::resident_chunks && nch <= Px3Layout<32>::resident_chunks)
    return launch_px3_co<32>(a, in_dtype, out_dtype, stream);
  // C_in > 128: streamed chunks over flattened tiles, when every frame's
  // bitmap and every frame's output planes are addressable by one buffer
  // resource each.
  if (nch > Px3Layout<32>::resident_chunks && a.n * (int64_t)a.hw_in * a.cwp * 4 < 0x7fffffffLL &&
      a.n * (int64_t)(a.c_out + 64) * a.hw_out * out_bytes < 0x7fffffffLL) {
    if (in_dtype == SF_F16) return launch_px3s_t<__half>(a, out_dtype, stream, dense);
    if (in_dtype == SF_BF16) return launch_px3s_t<__hip_bfloat16>(a, out_dtype, stream, dense);
    return launch_px3s_t<float>(a, out_dtype, stream, dense);
  }
  return launch_px3_co<64>(a, in_dtype, out_dtype, stream);
}

// Fused LIF: 32 output channels per workgroup.  The membrane shares the
// accumulator registers, and with 32 channels the weights of up to 128 input
// channels stay resident (config 4) and a sample's tiles spread over twice
// as many workgroups.
template <typename TIn, typename TOut>
int launch_px3_lif_t(const ConvArgs& a, hipStream_t stream) {
  // Up to 128 input channels: every weight row resident and the spikes
  // walked as 64-channel super-chunks (fewer rounds than 32-channel chunks:
  // a round count is the busiest lane's, which grows more slowly than the
  // mean).
  if (a.c_in <= 128 && a.cwp <= 4) return launch_px3w_to<TIn, TOut, 32, true>(a, stream);
  return launch_px3_t<TIn, TOut, 32, true>(a, 0, stream);
}

int launch_px3_lif(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  // Spike dtype: the input's, or f32 (the combinations sf_conv_lif_forward accepts).
  if (in_dtype == SF_F16)
    return out_dtype == SF_F32 ? launch_px3_lif_t<__half, float>(a, stream) : launch_px3_lif_t<__half, __half>(a, stream);
  if (in_dtype == SF_BF16)
    return out_dtype == SF_F32 ? launch_px3_lif_t<__hip_bfloat16, float>(a, stream)
                               : launch_px3_lif_t<__hip_bfloat16, __hip_bfloat16>(a, stream);
  return launch_px3_lif_t<float, float>(a, stream);
}

}  // namespace

bool px3_resident(const ConvArgs& a) {
  const int nch = (a.c_in + kPx3Ch - 1) / kPx3Ch;
  return nch <= Px3Layout<32>::resident_chunks;
}

bool px3_applicable(const ConvArgs& a) {
  // (A frame's bitmap must stay below 2 GB: px3_load_words addresses it
  // through a buffer resource and marks taps outside the frame with offset
  // 2^31.)
  return a.k == 3 && a.p == 1 && (a.s == 1 || a.s == 2) && a.c_out % 4 == 0 && a.cwp <= 64 &&
         a.n * (int64_t)((a.hw_out + 63) / 64) < (1ll << 30) && (int64_t)a.hw_in * a.cwp * 4 < (1ll << 31);
}

int launch_conv_px3(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  DenseQueue* dense = nullptr;
  timing_begin(K_PX3, stream);
  int rc = launch_px3_conv(a, in_dtype, out_dtype, stream, &dense);
  timing_end(K_PX3, stream);
  // The tiles the walk queued for the matrix cores, right after it.
  if (rc == (int)hipSuccess && dense != nullptr) rc = launch_conv_dense_mfma(a, dense, out_dtype, stream);
  return rc;
}

int launch_conv_lif_px3(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_LIF_PX3, stream);
  const int rc = launch_px3_lif(a, in_dtype, out_dtype, stream);
  timing_end(K_LIF_PX3, stream);
  return rc;
}

}  // namespace sf
