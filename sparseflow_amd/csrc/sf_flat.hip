// Stage 2 for 1x1 stride-1 convolutions: flat 64-pixel tiles, lane = pixel.
//
// One wavefront owns 64 consecutive pixels of one frame (a flat run of the
// h*w plane; no halo) for 64 output channels: lane = pixel, one accumulator
// register per output channel.  Each lane walks the set bits of its own
// pixel's bitmap words (a divergent loop: the wavefront runs as many rounds as
// its busiest pixel) and adds weight row ci, 64 output channels read from LDS
// as 16 x 16-byte pieces, to its accumulators.  No scalar-unit walk, no
// register transpose: the finished tile is stored one output channel per
// instruction, 64 consecutive pixels = one 256-byte run per channel plane.
//
// LDS layout: weight row ci of the workgroup's 64-channel group takes 512
// bytes, the row's 16 pieces written twice and rotated by (ci mod 16) pieces,
// so that a read of pieces k..k+15 (k = ci mod 16) returns the row in order
// with plain immediate offsets while lanes reading different rows spread over
// the LDS banks.  Chunks of 128 input channels (64 KB); with at most two
// chunks (C_in <= 256) they stay resident for the whole persistent launch and
// the wavefronts never synchronise, beyond that chunk c+1 streams into the
// second buffer (direct global->LDS loads) while chunk c is walked.
//
// The same kernel serves the sparse linear (ROWS = true): a "pixel" is a row
// of x [m, k] (k contiguous, one frame), non-binary values are read along
// the row and the lane's 64 outputs are one contiguous 256-byte run of the
// row-major y [m, c_out], written as 16-byte pieces.
//
// Output element (co, p) = bias[co] + its spikes summed by one lane in
// increasing ci: deterministic from run to run.
// Replaces the reference's sparse_conv1x1_nhwc_kernel_8x8/8x16
// (Kernels/conv2d.py:237-361) and its fused persistent 1x1 path
// (Kernels/conv2d.py:364-560) for these shapes.
#include "sf_tile.h"

namespace sf {

namespace {

constexpr int kPxChunkCh = 128;                            // input channels per weight chunk
constexpr int kPxChunkWords = kPxChunkCh / 32;             // bitmap words per chunk
constexpr int kPxRowBytes = 512;                           // one rotated, doubled weight row
constexpr int kPxChunkBytes = kPxChunkCh * kPxRowBytes;    // 64 KB

// Direct-to-LDS loads of weight chunk c (rows c*128 .. +127 of wt, channels
// co0 .. co0+63).  Each 1 KB unit is two rotated rows, one wavefront
// instruction: lane l carries row 2u + l/32, position q = l % 32 of that row,
// which holds the 16-byte piece (q - row) mod 16 (channels 4 * piece .. +3).
// Rows past C_in are skipped; channels past C_out read a valid but unrelated
// address whose values are never stored.
template <int NWAVES = kRowsWaves>
__device__ __forceinline__ void load_chunk_px(char* buf, const float* __restrict__ wt, int c, int c_in, int c_out,
                                              int co0, int wave, int lane) {
  const int rows = min(kPxChunkCh, c_in - c * kPxChunkCh);
  const int units = (rows + 1) / 2;
#pragma unroll
  for (int j = 0; j < kPxChunkBytes / 1024 / NWAVES; ++j) {
    const int u = wave + NWAVES * j;
    if (u < units) {
      const int r = 2 * u + (lane >> 5);
      const int piece = ((lane & 31) - r) & 15;
      const int row = c * kPxChunkCh + r;
      const int col = co0 + 4 * piece;
      const float* src = (row < c_in && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  }
}

// load_chunk_px by the nw wavefronts of a workgroup sized at run time.
__device__ __forceinline__ void load_chunk_px_nw(char* buf, const float* __restrict__ wt, int c, int c_in, int c_out,
                                                 int co0, int wave, int nw, int lane) {
  const int rows = min(kPxChunkCh, c_in - c * kPxChunkCh);
  const int units = (rows + 1) / 2;
  for (int u = wave; u < units; u += nw) {
    const int r = 2 * u + (lane >> 5);
    const int piece = ((lane & 31) - r) & 15;
    const int row = c * kPxChunkCh + r;
    const int col = co0 + 4 * piece;
    const float* src = (row < c_in && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
  }
}

// Bitmap words as a lane walks them: 64-bit (two channel words) except for
// single-word pixels.
template <int CW>
struct PxWord {
  typedef uint64_t type;
  static constexpr int count = CW / 2;
};
template <>
struct PxWord<1> {
  typedef uint32_t type;
  static constexpr int count = 1;
};

__device__ __forceinline__ int px_first_bit(uint32_t m) { return __builtin_ctz(m); }
__device__ __forceinline__ int px_first_bit(uint64_t m) { return __builtin_ctzll(m); }

// Add weight row r of the chunk, times xv, to the lane's 64 accumulators.
__device__ __forceinline__ void px_add_row(float (&acc)[64], const char* chunk, int r, float xv) {
  const float4* rp = reinterpret_cast<const float4*>(chunk + r * kPxRowBytes + ((r & 15) << 4));
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    // Groups of four pieces: the scheduler may not hoist more than 16
    // loaded registers ahead of their use (the accumulators take 64).
    if (s % 4 == 0) __builtin_amdgcn_sched_barrier(0);
    const float4 v = rp[s];
    acc[4 * s] = fmaf(xv, v.x, acc[4 * s]);
    acc[4 * s + 1] = fmaf(xv, v.y, acc[4 * s + 1]);
    acc[4 * s + 2] = fmaf(xv, v.z, acc[4 * s + 2]);
    acc[4 * s + 3] = fmaf(xv, v.w, acc[4 * s + 3]);
  }
}

// Store the lane's pixel for output channels 0 .. nco-1 of the group: one
// channel plane per instruction, 64 lanes = 64 consecutive pixels.
template <typename TOut>
__device__ __forceinline__ void px_store(const float (&acc)[64], TOut* __restrict__ yp, int hw, int nco) {
  if (nco >= 64) {
#pragma unroll
    for (int co = 0; co < 64; ++co) yp[(int64_t)co * hw] = from_f32<TOut>(acc[co]);
  } else {
#pragma unroll
    for (int co = 0; co < 64; ++co)
      if (co < nco) yp[(int64_t)co * hw] = from_f32<TOut>(acc[co]);
  }
}

// Row-major store: the lane's outputs co0 .. co0+nco-1 are contiguous
// (nco % 4 == 0).
template <typename TOut>
__device__ __forceinline__ void px_store_rows(const float (&acc)[64], TOut* __restrict__ yp, int nco) {
#pragma unroll
  for (int s = 0; s < 16; ++s)
    if (nco >= 64 || 4 * s < nco) store4<TOut>(yp + 4 * s, acc[4 * s], acc[4 * s + 1], acc[4 * s + 2], acc[4 * s + 3]);
}

// Dense-tile branch of the streamed 1x1 walk (C_in > 256: every chunk step
// ends at a barrier): a binary tile of which some pixel has kFlatDenseSpikes
// or more spikes among the first chunk's 128 channels (i.i.d. spikes at 1%
// density average 1.28 there; a 64-pixel tile reaches 10 with probability ~5e-5)
// holds its pass for several times an ordinary tile's walk.  Its run of
// output pixels goes to the matrix-core queue instead (k_conv_dense_mfma in
// its 1x1 form, launched right after on the same stream).
constexpr int kFlatDenseSpikes = 10;

template <int CW, typename TIn, bool ROWS>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_flat(ConvArgs a, const uint32_t* __restrict__ bits,
                                                               const uint32_t* __restrict__ flags,
                                                               const TIn* __restrict__ x,
                                                               const float* __restrict__ wt,
                                                               const float* __restrict__ bias_p,
                                                               void* __restrict__ y, int groups, int nchunks,
                                                               int out_dtype, DenseQueue* __restrict__ dq) {
  typedef typename PxWord<CW>::type WT;
  constexpr int NW = PxWord<CW>::count;          // walk words per pixel and chunk
  constexpr int BITS = 8 * (int)sizeof(WT);
  extern __shared__ __align__(16) char smem[];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6));  // tiles per pass
  const int blk = xcd_local_block((int)blockIdx.x, (int)gridDim.x);
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const int hw = a.hw_in;
  const int tpf = (hw + 63) / 64;
  const int total = (int)a.n * tpf;
  const int nblk = (int)(gridDim.x / groups);
  const bool resident = nchunks <= 2;
  // The group's bias in LDS: read per pass from global memory it would be a
  // vector load that waits for every store the wavefront still has in flight.
  __shared__ float s_bias[64];
  if (threadIdx.x < 64) {
    const int co = co0 + (int)threadIdx.x;
    s_bias[threadIdx.x] = (bias_p != nullptr && co < a.c_out) ? bias_p[co] : 0.f;
  }
  __syncthreads();

  if (resident) {
    for (int c = 0; c < nchunks; ++c)
      load_chunk_px_nw(smem + c * kPxChunkBytes, wt, c, a.c_in, a.c_out, co0, wave, nw, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // Passes of nw tiles.  With more than two chunks every wavefront takes
  // part in every barrier, including those of a pass past the end.
  for (int pass = (blk / groups); pass * nw < total; pass += nblk) {
    const int t = pass * nw + wave;
    const bool valid = t < total;
    const int frame = valid ? t / tpf : 0;
    const int p0 = valid ? (t - frame * tpf) * 64 : 0;
    const int npx = min(64, hw - p0);
    const bool mine = valid && lane < npx;  // this lane's pixel exists
    // Per-channel values (bias, store offsets) are formed in every pass,
    // not kept live across the loop: the accumulators need the registers.
    int hw_t = hw, c_out_t = a.c_out;
    asm volatile("" : "+s"(hw_t), "+s"(c_out_t));
    float acc[64];
#pragma unroll
    for (int co = 0; co < 64; ++co) acc[co] = s_bias[co];
    bool value = false;
    if (valid) {
      const int64_t c_a = p0 / a.chunk, c_b = (p0 + npx - 1) / a.chunk;
      const uint32_t* __restrict__ fl = flags + (int64_t)frame * a.chunks_per_frame;
      uint32_t f = 0u;
      for (int64_t q = c_a; q <= c_b; ++q) f |= fl[q];
      value = f != 0u;
    }
    bool walk = mine;
    if constexpr (!ROWS && CW == kPxChunkWords) {
      if (dq != nullptr && !resident && valid && !value) {
        uint32_t cnt = 0u;
        if (mine) {
          const uint32_t* __restrict__ bp = bits + ((int64_t)frame * hw + p0 + lane) * a.cwp;
#pragma unroll
          for (int j = 0; j < CW; ++j) cnt += (uint32_t)__popc(bp[j]);
        }
        if (__ballot(cnt >= (uint32_t)kFlatDenseSpikes) != 0ull) {
          uint32_t slot = 0u;
          if (lane == 0) slot = atomicAdd(&dq->count[grp], 1u);
          slot = __builtin_amdgcn_readfirstlane(slot);
          // A slot past the queue's capacity is not written (nor read); the
          // tile is walked.
          if (slot < (uint32_t)kDenseQueueCap) {
            if (lane == 0) {
              dq->start[grp][slot] = (uint32_t)((int64_t)frame * hw + p0);
              dq->npx[grp][slot] = (uint8_t)npx;
            }
            walk = false;
          }
        }
      }
    }
    // This lane's pixel (row), channel 0, and the distance between channels.
    const TIn* xp = ROWS ? x + (int64_t)(p0 + lane) * a.c_in : x + (int64_t)frame * a.c_in * hw + p0 + lane;
    const int64_t xcs = ROWS ? 1 : hw;
    if (!resident) {
      __syncthreads();  // the previous pass is done with both buffers
      load_chunk_px_nw(smem, wt, 0, a.c_in, a.c_out, co0, wave, nw, lane);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    for (int c = 0; c < nchunks; ++c) {
      // Stream chunk c+1 into the other buffer; it was last read during
      // chunk c-1, which every wavefront finished before the last barrier.
      if (!resident && c + 1 < nchunks)
        load_chunk_px_nw(smem + ((c + 1) & 1) * kPxChunkBytes, wt, c + 1, a.c_in, a.c_out, co0, wave, nw, lane);
      if (walk) {
        WT w[NW];
        const WT* __restrict__ bp =
            reinterpret_cast<const WT*>(bits + ((int64_t)frame * hw + p0 + lane) * a.cwp + c * CW);
#pragma unroll
        for (int j = 0; j < NW; ++j) w[j] = bp[j];
        const char* chunk = smem + (c & 1) * kPxChunkBytes;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          WT m = w[j];
          // One loop body for both paths (binary tiles multiply by exactly
          // 1): a second copy of the accumulator updates would double their
          // live ranges.
          while (m) {
            const int r = j * BITS + px_first_bit(m);
            m &= m - 1;
            float xv = 1.f;
            if (value) {
              xv = to_f32<TIn>(xp[(int64_t)(c * kPxChunkCh + r) * xcs]);
              // Waited for here, in the value path: otherwise every round's
              // products wait for all memory operations in flight (the next
              // chunk's streamed rows and bitmap words among them).
              __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
            }
            px_add_row(acc, chunk, r, xv);
          }
        }
      }
      if (!resident) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
    if (walk && ROWS) {
      const int64_t yb = (int64_t)(p0 + lane) * c_out_t + co0;
      const int nco = min(64, c_out_t - co0);
      if (out_dtype == SF_F16) px_store_rows(acc, static_cast<__half*>(y) + yb, nco);
      else if (out_dtype == SF_BF16) px_store_rows(acc, static_cast<__hip_bfloat16*>(y) + yb, nco);
      else px_store_rows(acc, static_cast<float*>(y) + yb, nco);
    } else if (walk) {
      const int64_t yb = ((int64_t)frame * c_out_t + co0) * hw_t + p0 + lane;
      const int nco = min(64, c_out_t - co0);
      if (out_dtype == SF_F16) px_store(acc, static_cast<__half*>(y) + yb, hw_t, nco);
      else if (out_dtype == SF_BF16) px_store(acc, static_cast<__hip_bfloat16*>(y) + yb, hw_t, nco);
      else px_store(acc, static_cast<float*>(y) + yb, hw_t, nco);
    }
  }
}

// Output spike map of the fused LIF variant (cwp words per pixel, chunk
// flags cleared): word w of pixel p of a frame at p * ps + w * ws words from
// the frame's start, (cwp, 1) pixel-major or (1, hw) as word planes.
struct FlatLifOut {
  uint32_t* bits;     // nullable
  uint32_t* flags;
  int cwp, chunk;
  int64_t cpf;        // flag chunks per frame
  // Nullable: a binary residual given by its pixel-major spike map (cwp
  // words per pixel), read instead of x2: two words per pixel instead of 64
  // values.
  const uint32_t* rbits;
  int ps, ws;
};

// Fused 1x1 conv + multi-step LIF: a tile of 64 pixels of one sample runs all
// T steps, the membrane carried in the accumulators between steps (seeded
// with the decay form, as the 3x3 fused kernel does); an optional second
// input x2 (a residual, same layout as the conv output) is added into the
// current of each step.  Per step the lane stores its pixel's 64 spikes
// (one channel per instruction) and, when requested, the two 32-channel
// bitmap words of those spikes, so the next sparse convolution needs no
// prescan.  The membrane after step T goes to v_out.
// Four or eight wavefronts per workgroup (the membrane-carrying accumulators
// and the step loop need more than the 128 registers a 16-wavefront group
// allows).

// VEC: C_out % 64 == 0 and H*W % 4 == 0 (four-pixel vector spike stores).
// XV: a residual given by its values (x2); without it the 64 prefetch
// registers of the residual are not allocated.
// NWV: wavefronts per workgroup (4 where the weights are small enough for
// three workgroups per CU, else 8).
template <int CW, typename TIn, typename TOut, bool VEC, bool XV, int NWV>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(XV ? 2 : 3, 8))) void k_conv_flat_lif(ConvArgs a, const uint32_t* __restrict__ bits,
                                                                   const uint32_t* __restrict__ flags,
                                                                   const TIn* __restrict__ x,
                                                                   const float* __restrict__ wt,
                                                                   const float* __restrict__ bias_p,
                                                                   const TIn* __restrict__ x2,
                                                                   TOut* __restrict__ spikes, FlatLifOut o,
                                                                   int groups, int nchunks) {
  typedef typename PxWord<CW>::type WT;
  constexpr int NW = PxWord<CW>::count;
  constexpr int BITS = 8 * (int)sizeof(WT);
  extern __shared__ __align__(16) char smem[];
  const int lane0 = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = xcd_local_block((int)blockIdx.x, (int)gridDim.x);
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const int hw = a.hw_in;
  const int tpf = (hw + 63) / 64;
  const int total = (int)a.n * tpf;  // a.n = samples; the T steps run inside a tile
  const int nblk = (int)(gridDim.x / groups);
  const bool resident = nchunks <= 2;
  const LifCoef L = lif_coef(a);
  __shared__ float s_seed[64];  // vr_term + bias of the group's channels
  if (threadIdx.x < 64) {
    const int c = min(co0 + (int)threadIdx.x, a.c_out - 1);
    s_seed[threadIdx.x] = L.vr_term + (bias_p != nullptr ? bias_p[c] : 0.f);
  }
  __syncthreads();

  if (resident) {
    for (int c = 0; c < nchunks; ++c)
      load_chunk_px<NWV>(smem + c * kPxChunkBytes, wt, c, a.c_in, a.c_out, co0, wave, lane0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (int pass = (blk / groups); pass * NWV < total; pass += nblk) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int t = pass * NWV + wave;
    const bool valid = t < total;
    const int sample = valid ? t / tpf : 0;
    const int p0 = valid ? (t - sample * tpf) * 64 : 0;
    const int npx = min(64, hw - p0);
    const bool mine = valid && lane < npx;
    int hw_t = hw, c_out_t = a.c_out;
    asm volatile("" : "+s"(hw_t), "+s"(c_out_t));
    int nco = VEC ? 64 : min(64, c_out_t - co0);
    // Loads use the pixel and channel clamped into range (valid addresses;
    // values of channels past C_out are never stored), stores are guarded.
    const int lc = min(lane, npx - 1);
    float acc[64];
#pragma unroll
    for (int co = 0; co < 64; ++co) acc[co] = 0.f;
    // Per-sample / per-frame planes [c_out, hw] through buffer descriptors.
    const uint32_t vplane = (uint32_t)c_out_t * (uint32_t)hw_t * 4u;
    if (a.v_init != nullptr && valid) {
      const auto vr = buf_rsrc(a.v_init + (int64_t)sample * c_out_t * hw_t, vplane);
#pragma unroll
      for (int co = 0; co < 64; ++co) acc[co] = BufIO<float>::load(vr, (p0 + lc) * 4, (co0 + min(co, nco - 1)) * hw_t * 4);
    }
    // Step st+1's residual, first-chunk bitmap words and flag are loaded one
    // step ahead.  The vector memory counter retires in issue order, so with
    // one store per channel plane (64 per step) they are issued before the
    // stores; the vector-store path issues them after its 18 stores, which
    // keeps the residual registers free while the store values are built.
    // The residual stays in its input type until it is added (a conversion
    // next to the load would wait for it).
    TIn res[XV ? 64 : 1];
    WT bw[NW];
    uint32_t fv = 0u, rw0 = 0u, rw1 = 0u;
    auto fetch = [&](int st) {
      const int64_t frame = (int64_t)st * a.n + sample;
      if (o.rbits != nullptr) {
        const uint32_t* rp = o.rbits + (frame * hw_t + p0 + lc) * o.cwp + co0 / 32;
        rw0 = rp[0];
        rw1 = co0 / 32 + 1 < o.cwp ? rp[1] : 0u;
      } else if (XV && x2 != nullptr) {
        constexpr int B = (int)sizeof(TIn);
        const auto rr = buf_rsrc(x2 + frame * c_out_t * hw_t, (uint32_t)c_out_t * (uint32_t)hw_t * B);
#pragma unroll
        for (int co = 0; co < 64; ++co) res[co] = BufIO<TIn>::load(rr, (p0 + lc) * B, (co0 + min(co, nco - 1)) * hw_t * B);
      }
      const WT* __restrict__ bp = reinterpret_cast<const WT*>(bits + (frame * hw + p0 + lc) * a.cwp);
#pragma unroll
      for (int j = 0; j < NW; ++j) bw[j] = bp[j];
      // A 64-pixel tile lies in one flag chunk (chunks are multiples of 64).
      fv = flags[frame * a.chunks_per_frame + p0 / a.chunk];
    };
    if (valid) fetch(0);
    for (int st = 0; st < a.T; ++st) {
      const int64_t frame = (int64_t)st * a.n + sample;
      // Keep the per-channel offset arithmetic inside the step (hoisted, its
      // 64 scalar offsets would spill).
      asm volatile("" : "+s"(hw_t), "+s"(c_out_t));
      nco = VEC ? 64 : min(64, c_out_t - co0);
      lif_seed_lds<64>(acc, L, s_seed);
      if (o.rbits != nullptr) {
        // The same sums as adding the 0 / 1 values.
#pragma unroll
        for (int co = 0; co < 64; ++co) acc[co] += (((co < 32 ? rw0 : rw1) >> (co & 31)) & 1u) ? 1.f : 0.f;
      } else if (XV && x2 != nullptr) {
#pragma unroll
        for (int co = 0; co < 64; ++co) acc[co] += to_f32<TIn>(res[co]);
      }
      const bool value = valid && fv != 0u;
      const TIn* xp = x + frame * a.c_in * hw + p0 + lane;
      if (!resident) {
        __syncthreads();  // the previous step/pass is done with both buffers
        // Streaming addresses formed here (hoisted, they would be spilled).
        int ll = lane;
        asm volatile("" : "+v"(ll));
        load_chunk_px<NWV>(smem, wt, 0, a.c_in, a.c_out, co0, wave, ll);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
      for (int c = 0; c < nchunks; ++c) {
        if (!resident && c + 1 < nchunks) {
          int ll = lane;
          asm volatile("" : "+v"(ll));
          load_chunk_px<NWV>(smem + ((c + 1) & 1) * kPxChunkBytes, wt, c + 1, a.c_in, a.c_out, co0, wave, ll);
        }
        if (mine) {
          WT w[NW];
          if (c == 0) {
#pragma unroll
            for (int j = 0; j < NW; ++j) w[j] = bw[j];
          } else {
            const WT* __restrict__ bp = reinterpret_cast<const WT*>(bits + (frame * hw + p0 + lane) * a.cwp + c * CW);
#pragma unroll
            for (int j = 0; j < NW; ++j) w[j] = bp[j];
          }
          const char* chunk = smem + (resident ? c : (c & 1)) * kPxChunkBytes;
#pragma unroll
          for (int j = 0; j < NW; ++j) {
            WT m = w[j];
            while (m) {
              const int r = j * BITS + px_first_bit(m);
              m &= m - 1;
              float xv = 1.f;
              if (value) {
                xv = to_f32<TIn>(xp[(int64_t)(c * kPxChunkCh + r) * hw]);
                // Waited for in the value path only (the step's prefetches
                // stay in flight during the bitmap path's rounds).
                __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
              }
              px_add_row(acc, chunk, r, xv);
            }
          }
        }
        if (!resident) {
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
        }
      }
      // H, spike, reset: the spikes are collected as two 32-channel words
      // (the bitmap words of the spike map), then stored from them; the
      // membrane stays in acc.
      uint32_t w0 = 0u, w1 = 0u;
#pragma unroll
      for (int co = 0; co < 64; ++co) {
        const float h = L.decay_input ? acc[co] * L.inv_tau : acc[co];
        const bool fire = h >= L.v_th;
        if (co < 32) w0 |= (fire ? 1u : 0u) << co;
        else w1 |= (fire ? 1u : 0u) << (co - 32);
        acc[co] = L.hard ? (fire ? L.v_reset : h) : h - (fire ? L.v_th : 0.f);
      }
      if (nco < 32) w0 &= (1u << nco) - 1u;
      if (nco < 64) w1 &= nco > 32 ? (1u << (nco - 32)) - 1u : 0u;
      if (!VEC && valid && st + 1 < a.T) fetch(st + 1);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (VEC) {
        // Lane l stores pixels p0 + 4*(l & 15) .. +3 of channel 4*i + (l >> 4),
        // i = 0..15: sixteen vector stores per step instead of 64 (the four
        // pixels' spike words are gathered from their lanes).  npx is a
        // multiple of 4 here.
        const int src = 4 * (lane & 15);
        uint32_t g0[4], g1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          g0[j] = __shfl(w0, src + j);
          g1[j] = __shfl(w1, src + j);
        }
        if (valid && src < npx) {
          constexpr int B = (int)sizeof(TOut);
          const auto sr = buf_rsrc(spikes + frame * c_out_t * hw_t, (uint32_t)c_out_t * (uint32_t)hw_t * B);
          const int cq = lane >> 4;
          const int vo = ((co0 + cq) * hw_t + p0 + src) * B;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int sh = 4 * (i & 7) + cq;
            const uint32_t* g = i < 8 ? g0 : g1;
            const uint32_t q = ((g[0] >> sh) & 1u) | (((g[1] >> sh) & 1u) << 1) | (((g[2] >> sh) & 1u) << 2) |
                               (((g[3] >> sh) & 1u) << 3);
            store_bits4<TOut>(q, sr, vo + 4 * i * hw_t * B);
          }
        }
      } else if (mine) {  // one channel plane per store
        constexpr int B = (int)sizeof(TOut);
        const auto sr = buf_rsrc(spikes + frame * c_out_t * hw_t, (uint32_t)c_out_t * (uint32_t)hw_t * B);
        const int vo = (p0 + lane) * B;
        if (nco >= 64) {
#pragma unroll
          for (int co = 0; co < 64; ++co) {
            // Groups of eight: the residual loads in flight already hold 64
            // registers, so the 0/1 values are not all materialised first.
            if (co % 8 == 0) __builtin_amdgcn_sched_barrier(0);
            BufIO<TOut>::store(from_f32<TOut>((float)(((co < 32 ? w0 : w1) >> (co & 31)) & 1u)), sr, vo,
                               (co0 + co) * hw_t * B);
          }
        } else {
          for (int co = 0; co < nco; ++co)
            BufIO<TOut>::store(from_f32<TOut>((float)(((co < 32 ? w0 : w1) >> (co & 31)) & 1u)), sr, vo,
                               (co0 + co) * hw_t * B);
        }
      }
      if (o.bits != nullptr && mine) {
        uint32_t* ob = o.bits + frame * hw_t * o.cwp + (int64_t)(p0 + lane) * o.ps;
        const int w_0 = co0 / 32;
        ob[(int64_t)w_0 * o.ws] = w0;
        if (w_0 + 1 < o.cwp) ob[(int64_t)(w_0 + 1) * o.ws] = w1;
        if (grp == groups - 1)  // the words past the last group's channels
          for (int wd = w_0 + 2; wd < o.cwp; ++wd) ob[(int64_t)wd * o.ws] = 0u;
      }
      if (o.bits != nullptr && valid && grp == 0 && lane == 0 && p0 % o.chunk == 0)
        o.flags[frame * o.cpf + p0 / o.chunk] = 0u;  // spikes are binary
      if (VEC && valid && st + 1 < a.T) {
        __builtin_amdgcn_sched_barrier(0);
        fetch(st + 1);
      }
    }
    if (mine) {
      const auto vr = buf_rsrc(a.v_out + (int64_t)sample * c_out_t * hw_t, vplane);
      if (nco >= 64) {
#pragma unroll
        for (int co = 0; co < 64; ++co) BufIO<float>::store(acc[co], vr, (p0 + lane) * 4, (co0 + co) * hw_t * 4);
      } else {
#pragma unroll
        for (int co = 0; co < 64; ++co)
          if (co < nco) BufIO<float>::store(acc[co], vr, (p0 + lane) * 4, (co0 + co) * hw_t * 4);
      }
    }
  }
}

template <int CW, typename TIn, typename TOut, bool VEC, bool XV, int NWV>
int launch_flat_lif_t(const ConvArgs& a, const void* x2, const FlatLifOut& o, hipStream_t stream) {
  const int groups = (a.c_out + 63) / 64;
  const int nchunks = CW < kPxChunkWords ? 1 : a.cwp / kPxChunkWords;
  const int last_units = (min(kPxChunkCh, a.c_in - (nchunks - 1) * kPxChunkCh) + 1) / 2;
  const size_t lds = nchunks <= 2 ? (size_t)(nchunks - 1) * kPxChunkBytes + (size_t)last_units * 1024
                                  : (size_t)2 * kPxChunkBytes;
  const int64_t tiles = a.n * (int64_t)((a.hw_in + 63) / 64);
  const int64_t need = (tiles + NWV - 1) / NWV;
  const int64_t cap = (int64_t)num_cus() * (NWV == 4 ? 3 : 1);  // resident workgroups
  const int per_group = (int)(need < cap ? need : cap);
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_flat_lif<CW, TIn, TOut, VEC, XV, NWV>;
  // The kernel also holds 256 B of static LDS (the per-channel seed).
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes - 1024);
  if (e != (int)hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * NWV), lds, stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, static_cast<const TIn*>(x2),
                     static_cast<TOut*>(a.y), o, groups, nchunks);
  return (int)hipGetLastError();
}

template <int CW, typename TIn, typename TOut>
int launch_flat_lif_v(const ConvArgs& a, const void* x2, const FlatLifOut& o, hipStream_t stream) {
  const bool vec = a.c_out % 64 == 0 && a.hw_in % 4 == 0;
  const bool xv = x2 != nullptr && o.rbits == nullptr;
  // Three 4-wave workgroups per CU when their weights fit three times in LDS
  // (C_in <= 96) and no value residual takes the registers.
  const bool small = !xv && a.c_in <= 96;
  if (vec) {
    if (xv) return launch_flat_lif_t<CW, TIn, TOut, true, true, 8>(a, x2, o, stream);
    return small ? launch_flat_lif_t<CW, TIn, TOut, true, false, 4>(a, x2, o, stream)
                 : launch_flat_lif_t<CW, TIn, TOut, true, false, 8>(a, x2, o, stream);
  }
  if (xv) return launch_flat_lif_t<CW, TIn, TOut, false, true, 8>(a, x2, o, stream);
  return small ? launch_flat_lif_t<CW, TIn, TOut, false, false, 4>(a, x2, o, stream)
               : launch_flat_lif_t<CW, TIn, TOut, false, false, 8>(a, x2, o, stream);
}

template <typename TIn, typename TOut>
int launch_flat_lif_d(const ConvArgs& a, const void* x2, const FlatLifOut& o, hipStream_t stream) {
  switch (a.cwp) {
    case 1: return launch_flat_lif_v<1, TIn, TOut>(a, x2, o, stream);
    case 2: return launch_flat_lif_v<2, TIn, TOut>(a, x2, o, stream);
    default: return launch_flat_lif_v<4, TIn, TOut>(a, x2, o, stream);
  }
}

template <int CW, typename TIn, bool ROWS>
int launch_flat_t(const ConvArgs& a, int out_dtype, hipStream_t stream, DenseQueue** dense) {
  const int groups = (a.c_out + 63) / 64;
  const int nchunks = CW < kPxChunkWords ? 1 : a.cwp / kPxChunkWords;
  // Resident: the chunks up to the last one's used 1 KB units; streamed: two
  // full buffers.
  const int last_units = (min(kPxChunkCh, a.c_in - (nchunks - 1) * kPxChunkCh) + 1) / 2;
  const size_t lds = nchunks <= 2 ? (size_t)(nchunks - 1) * kPxChunkBytes + (size_t)last_units * 1024
                                  : (size_t)2 * kPxChunkBytes;
  const int64_t tiles = a.n * (int64_t)((a.hw_in + 63) / 64);
  // Every CU makes the same number of passes (workgroup size from the
  // wave-tile count).
  const int nw = even_pass_waves(tiles * groups);
  const int64_t passes = (tiles * groups + (int64_t)num_cus() * nw - 1) / ((int64_t)num_cus() * nw);
  const int64_t per_group = (tiles + (int64_t)nw * passes - 1) / ((int64_t)nw * passes);
  const int grid = (int)(groups * (per_group > 0 ? per_group : 1));
  constexpr auto kern = k_conv_flat<CW, TIn, ROWS>;
  // 1 KB of the LDS is left to the kernel's static arrays.
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes - 1024);
  if (e != (int)hipSuccess) return e;
  // The dense-tile queue for the streamed conv (not the Linear), when entries
  // (a run's first pixel of the flattened axis, 31 bits) can address it.
  DenseQueue* dq = !ROWS && CW == kPxChunkWords && nchunks > 2 && groups <= kDenseQueueGroups &&
                           a.n * (int64_t)a.hw_in < (1ll << 31)
                       ? dense_queue_for(stream)
                       : nullptr;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), lds, stream, a, a.bits, a.flags,
                     static_cast<const TIn*>(a.x), a.wt, a.bias, a.y, groups, nchunks, out_dtype, dq);
  const int rc = (int)hipGetLastError();
  if (rc == (int)hipSuccess && dense != nullptr) *dense = dq;
  return rc;
}

template <typename TIn, bool ROWS>
int launch_flat_d(const ConvArgs& a, int out_dtype, hipStream_t stream, DenseQueue** dense = nullptr) {
  switch (a.cwp) {
    case 1: return launch_flat_t<1, TIn, ROWS>(a, out_dtype, stream, dense);
    case 2: return launch_flat_t<2, TIn, ROWS>(a, out_dtype, stream, dense);
    default: return launch_flat_t<4, TIn, ROWS>(a, out_dtype, stream, dense);
  }
}

}  // namespace

bool flat_applicable(const ConvArgs& a) {
  return a.k == 1 && a.s == 1 && a.p == 0 && a.h_out == a.h_in && a.w_out == a.w_in && a.c_out % 4 == 0 &&
         a.n * (int64_t)((a.hw_in + 63) / 64) < (1ll << 30);
}

int launch_conv_flat(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  DenseQueue* dense = nullptr;
  timing_begin(K_FLAT, stream);
  int rc = in_dtype == SF_F16    ? launch_flat_d<__half, false>(a, out_dtype, stream, &dense)
           : in_dtype == SF_BF16 ? launch_flat_d<__hip_bfloat16, false>(a, out_dtype, stream, &dense)
                                 : launch_flat_d<float, false>(a, out_dtype, stream, &dense);
  timing_end(K_FLAT, stream);
  // The tiles the walk queued for the matrix cores, right after it.
  if (rc == (int)hipSuccess && dense != nullptr) rc = launch_conv_dense_mfma(a, dense, out_dtype, stream);
  return rc;
}

int launch_linear_flat(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  timing_begin(K_LINEAR, stream);
  const int rc = in_dtype == SF_F16    ? launch_flat_d<__half, true>(a, out_dtype, stream)
                 : in_dtype == SF_BF16 ? launch_flat_d<__hip_bfloat16, true>(a, out_dtype, stream)
                                       : launch_flat_d<float, true>(a, out_dtype, stream);
  timing_end(K_LINEAR, stream);
  return rc;
}

int launch_conv_lif_flat(const ConvArgs& a, int in_dtype, int out_dtype, const void* x2, const uint32_t* res_bits,
                         uint32_t* out_bits, uint32_t* out_flags, int out_cwp, int out_planes, int out_chunk,
                         int64_t out_cpf, hipStream_t stream) {
  const int hw_out = a.h_out * a.w_out;
  FlatLifOut o{out_bits, out_flags, out_cwp, out_chunk, out_cpf, res_bits, out_planes ? 1 : out_cwp,
               out_planes ? hw_out : 1};
  if (a.chunk <= 0 || a.chunk % 64 != 0) return (int)hipErrorInvalidValue;  // one flag per 64-pixel tile
  timing_begin(K_LIF_FLAT, stream);
  int rc;
  if (in_dtype == SF_F16)
    rc = out_dtype == SF_F32 ? launch_flat_lif_d<__half, float>(a, x2, o, stream)
                             : launch_flat_lif_d<__half, __half>(a, x2, o, stream);
  else if (in_dtype == SF_BF16)
    rc = out_dtype == SF_F32 ? launch_flat_lif_d<__hip_bfloat16, float>(a, x2, o, stream)
                             : launch_flat_lif_d<__hip_bfloat16, __hip_bfloat16>(a, x2, o, stream);
  else
    rc = launch_flat_lif_d<float, float>(a, x2, o, stream);
  timing_end(K_LIF_FLAT, stream);
  return rc;
}

}  // namespace sf
