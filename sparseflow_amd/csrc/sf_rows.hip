// Stage 2, K-chunked row-band formulation for 3x3 stride-1 convolutions on
// 28- and 14-wide frames whose weights do not fit LDS (C_in > 64): lane =
// output channel, weights streamed through LDS in chunks of 32 input
// channels (k_conv_rows_kc below).
#include "sf_tile.h"

namespace sf {

namespace {

// ---------------------------------------------------------------------------
// K-chunked variant for layers whose weights do not fit LDS (C_in > 64).
//
// Tile = TH full rows of a W-wide frame (TH*W <= 64 output pixels, contiguous
// in the output plane), lane = output channel.  Weights are consumed in
// chunks of one 32-channel bitmap word (32 ci x 9 taps x 64 co = 72 KB),
// double-buffered in LDS: while the workgroup's 16 wavefronts walk chunk c
// from one buffer, chunk c+1 streams into the other with direct global->LDS
// loads.  One barrier per chunk.  With at most two chunks both stay resident
// and the wavefronts never synchronise.
// ---------------------------------------------------------------------------

constexpr int kChunkBytes = 32 * 9 * 64 * 4;  // one chunk of weights: 72 KB = 72 units of 1 KB

// Issue the direct-to-LDS loads of weight chunk c into `buf`.  Each 1 KB unit
// (4 weight rows x 64 channels) is one wavefront instruction: lane l carries
// row 4u + l/16, channels 4*(l%16) .. +3.  Rows past C_in and channels past
// C_out read a valid but unrelated address; those values are never used.
__device__ __forceinline__ void load_chunk(char* buf, const float* __restrict__ wt, int c, int krows, int c_out,
                                           int co0, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < (kChunkBytes / 1024 + kRowsWaves - 1) / kRowsWaves; ++j) {
    const int u = wave + kRowsWaves * j;
    if (u < kChunkBytes / 1024) {
      const int row = c * (32 * 9) + u * 4 + (lane >> 4);
      const int col = co0 + 4 * (lane & 15);
      const float* src = (row < krows && col < c_out) ? wt + (int64_t)row * c_out + col : wt;
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(buf + u * 1024), 16, 0, 0);
    }
  }
}

struct KcTile {
  // The chunk's bitmap words of the (TH + 2) x W halo positions, position p
  // in lane p & 63 of vw0 (p < 64) or vw1: fetched with two vector loads and
  // read on the scalar unit with readlane at compile-time lanes.
  uint32_t vw0, vw1;
  const void* x;            // x plane of the frame (value path)
  int64_t xrow;             // element offset of input row oh0 - 1 within a channel plane
  const char* wlb;          // LDS weight chunk + lane offset
  int oh0, h, cwp, hw, in_dtype, c0;  // c0 = first channel of the chunk
  bool value;               // tile reads non-binary inputs: multiply by x
};

// Spikes of halo position (IA, IB) (input row oh0-1+IA, column IB) whose
// chunk word is m.  Every weight row lands in a compile-time accumulator;
// binary tiles multiply by exactly 1.
template <int TH, int W, int IA, int IB>
__device__ __forceinline__ void kc_position(float (&acc)[64], uint32_t m, const KcTile& k) {
  while (m) {
    const int bit = __builtin_ctz(m);
    m &= m - 1;
    float xv = 1.f;
    if (k.value) xv = load_x(k.x, k.in_dtype, (int64_t)(k.c0 + bit) * k.hw + k.xrow + IA * W + IB);
    const char* base = k.wlb + bit * (9 * 256);
    // All of the spike's weight rows are read before the first FMA, so their
    // LDS round trips overlap (one wait per spike, not one per pair of rows).
    float wv[9];
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      const int r = IA - kh;
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        const int xo = IB + 1 - kw;
        wv[kh * 3 + kw] = (r < 0 || r >= TH || xo < 0 || xo >= W)
                              ? 0.f
                              : *reinterpret_cast<const float*>(base + (kh * 3 + kw) * 256);
      }
    }
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      const int r = IA - kh;
      if (r < 0 || r >= TH) continue;
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        const int xo = IB + 1 - kw;
        if (xo < 0 || xo >= W) continue;
        acc[r * W + xo] = fmaf(xv, wv[kh * 3 + kw], acc[r * W + xo]);
      }
    }
  }
}

template <int TH, int W, int IA, int B0, int U, int NB>
__device__ __forceinline__ void kc_batch_walk(float (&acc)[64], const uint32_t (&mw)[8], const KcTile& k) {
  if constexpr (U < NB) {
    kc_position<TH, W, IA, B0 + U>(acc, mw[U], k);
    kc_batch_walk<TH, W, IA, B0, U + 1, NB>(acc, mw, k);
  }
}

template <int P>
__device__ __forceinline__ uint32_t kc_word(const KcTile& k) {
  static_assert(P < 128, "halo positions fit two words per lane");
  return __builtin_amdgcn_readlane(P < 64 ? k.vw0 : k.vw1, P & 63);
}

template <int P, int U, int NB>
__device__ __forceinline__ void kc_fill(uint32_t (&mw)[8], const KcTile& k) {
  if constexpr (U < NB) {
    mw[U] = kc_word<P + U>(k);
    kc_fill<P, U + 1, NB>(mw, k);
  }
}

template <int TH, int W, int IA, int B0>
__device__ __forceinline__ void kc_row(float (&acc)[64], const KcTile& k) {
  if constexpr (B0 < W) {
    constexpr int NB = (W - B0) < 8 ? (W - B0) : 8;
    uint32_t mw[8];
    kc_fill<IA * W + B0, 0, NB>(mw, k);
    kc_batch_walk<TH, W, IA, B0, 0, NB>(acc, mw, k);
    kc_row<TH, W, IA, B0 + 8>(acc, k);
  }
}

template <int TH, int W, int IA>
__device__ __forceinline__ void kc_rows(float (&acc)[64], const KcTile& k) {
  if constexpr (IA < TH + 2) {
    const int ih = k.oh0 - 1 + IA;
    if (ih >= 0 && ih < k.h) kc_row<TH, W, IA, 0>(acc, k);
    kc_rows<TH, W, IA + 1>(acc, k);
  }
}

// Chunk c's words of the tile's halo positions (rows oh0 - 1 .. oh0 + TH of
// the frame; rows outside it read position 0 and come back as 0).  Word c
// of pixel q at q * ps + c * ws words from the frame's start: with word
// planes (ps = 1) the 64 lanes of a load read one run.
template <int TH, int W>
__device__ __forceinline__ void kc_load_words(uint32_t& v0, uint32_t& v1, const uint32_t* __restrict__ fbits,
                                              int oh0, int h, int ps, int ws, int lane, int c) {
  constexpr int NP = (TH + 2) * W;
  const int p0 = lane, p1 = 64 + lane;
  const int ih0 = oh0 - 1 + p0 / W, ih1 = oh0 - 1 + p1 / W;
  const bool ok0 = p0 < NP && ih0 >= 0 && ih0 < h, ok1 = p1 < NP && ih1 >= 0 && ih1 < h;
  const int64_t q0 = ok0 ? (int64_t)(oh0 - 1) * W + p0 : 0, q1 = ok1 ? (int64_t)(oh0 - 1) * W + p1 : 0;
  v0 = fbits[q0 * ps + (int64_t)c * ws];
  v1 = fbits[q1 * ps + (int64_t)c * ws];
  // Positions outside the halo or the frame hold no spikes (the walk never
  // reads them; the dense-tile branch counts every lane).
  v0 = ok0 ? v0 : 0u;
  v1 = ok1 ? v1 : 0u;
}

// Dense-tile branch of the row kernel: a binary tile whose first chunk (32
// input channels) holds kRowsDenseSpikes or more spikes in its halo rows
// (3-4x the mean at 1% density, 10+ standard deviations above it for i.i.d.
// spikes) is not walked.  Its walk would last several times an ordinary
// tile's, and since every chunk step ends at a barrier it would hold its
// whole pass: live spikes burst in a few time steps, and a pass covers
// consecutive frames of one step.  The tile's run of output pixels (TH rows
// of one frame, at most 64 pixels, contiguous on the flattened (frame,
// pixel) axis) goes to the matrix-core queue instead (k_conv_dense_mfma,
// launched right after on the same stream), which computes the 64 pixels
// from the run's first and stores the run's own.  A binary tile's halo rows
// are all the input rows those pixels read.
constexpr int kRowsDenseSpikes = 96;

template <int TH, int W>
__global__ __launch_bounds__(64 * kRowsWaves) void k_conv_rows_kc(ConvArgs a, const uint32_t* __restrict__ bits,
                                                                  const uint32_t* __restrict__ flags,
                                                                  const void* __restrict__ x,
                                                                  const float* __restrict__ wt,
                                                                  const float* __restrict__ bias_p,
                                                                  void* __restrict__ y, int groups, int nchunks,
                                                                  int in_dtype, int out_dtype,
                                                                  DenseQueue* __restrict__ dq) {
  // Launched only for planes with h*w % 4 == 0, so every tile's run (TH*W, or
  // an even number of 14-wide rows for the last tile) is whole quads.
  static_assert(TH * W <= 64 && (TH * W) % 4 == 0, "tile must be a whole number of quads within 64 pixels");
  extern __shared__ __align__(16) char smem[];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = (int)blockIdx.x;
  const int grp = blk % groups;
  const int co0 = grp * 64;
  const int krows = a.c_in * 9;
  const float bias = (bias_p != nullptr && co0 + lane < a.c_out) ? bias_p[co0 + lane] : 0.f;
  const int h = a.h_in;
  const int tpf = (h + TH - 1) / TH;
  const int total = (int)a.n * tpf;
  const int nblk = (int)(gridDim.x / groups);
  const bool resident = nchunks <= 2;
  const int in_size = in_dtype == SF_F32 ? 4 : 2;

  if (resident) {
    for (int c = 0; c < nchunks; ++c) load_chunk(smem + c * kChunkBytes, wt, c, krows, a.c_out, co0, wave, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // Passes of kRowsWaves tiles.  With more than two chunks every wavefront
  // takes part in every barrier, including those of a pass past the end.
  for (int pass = (blk / groups); pass * kRowsWaves < total; pass += nblk) {
    const int t = pass * kRowsWaves + wave;
    const bool valid = t < total;
    const int frame = valid ? t / tpf : 0;
    const int oh0 = valid ? (t - frame * tpf) * TH : 0;
    float acc[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) acc[i] = i < TH * W ? bias : 0.f;
    KcTile k;
    k.oh0 = oh0;
    k.h = h;
    k.cwp = a.cwp;
    k.hw = a.hw_in;
    k.in_dtype = in_dtype;
    k.x = static_cast<const char*>(x) + (int64_t)frame * a.c_in * a.hw_in * in_size;
    k.xrow = (int64_t)(oh0 - 1) * W;
    k.value = valid && rows_value_path(a, flags, frame, oh0 - 1, oh0 + TH);
    // Chunk 0's halo words; chunk c+1's are requested while chunk c is walked.
    const uint32_t* __restrict__ fbits = bits + (int64_t)frame * a.hw_in * a.cwp;
    uint32_t nw0 = 0u, nw1 = 0u;
    if (valid) kc_load_words<TH, W>(nw0, nw1, fbits, oh0, h, a.bm_ps, a.bm_ws, lane, 0);
    bool walk = valid;
    if (dq != nullptr && valid && !k.value) {
      int cnt = __popc(nw0) + __popc(nw1);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
      // Every lane holds the sum; read it as a scalar so that the walk below
      // stays a uniform branch.
      cnt = __builtin_amdgcn_readfirstlane(cnt);
      if (cnt >= kRowsDenseSpikes) {
        uint32_t slot = 0u;
        if (lane == 0) slot = atomicAdd(&dq->count[grp], 1u);
        slot = __builtin_amdgcn_readfirstlane(slot);
        // A slot past the queue's capacity is not written (nor read); the
        // tile is walked.
        if (slot < (uint32_t)kDenseQueueCap) {
          if (lane == 0) {
            dq->start[grp][slot] = (uint32_t)((int64_t)frame * a.hw_out + (int64_t)oh0 * W);
            dq->npx[grp][slot] = (uint8_t)(min(TH, h - oh0) * W);
          }
          walk = false;
        }
      }
    }
    if (!resident) {
      __syncthreads();  // the previous pass is done with both buffers
      load_chunk(smem, wt, 0, krows, a.c_out, co0, wave, lane);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    for (int c = 0; c < nchunks; ++c) {
      // Stream chunk c+1 into the other buffer; it was last read during
      // chunk c-1, which every wavefront finished before the last barrier.
      if (!resident && c + 1 < nchunks)
        load_chunk(smem + ((c + 1) & 1) * kChunkBytes, wt, c + 1, krows, a.c_out, co0, wave, lane);
      if (walk) {
        k.vw0 = nw0;
        k.vw1 = nw1;
        if (c + 1 < nchunks) kc_load_words<TH, W>(nw0, nw1, fbits, oh0, h, a.bm_ps, a.bm_ws, lane, c + 1);
        k.c0 = c * 32;
        k.wlb = smem + (c & 1) * kChunkBytes + lane * 4;
        kc_rows<TH, W, 0>(acc, k);
      }
      if (!resident) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
    if (walk) {
      const int npx = min(TH, h - oh0) * W;
      butterfly<1, 16>(acc, lane);
      butterfly<2, 16>(acc, lane);
      butterfly<4, 16>(acc, lane);
      butterfly<8, 16>(acc, lane);
      if (out_dtype == SF_F16) tile_store<__half>(acc, y, a, frame, co0, oh0 * W, npx, lane);
      else if (out_dtype == SF_BF16) tile_store<__hip_bfloat16>(acc, y, a, frame, co0, oh0 * W, npx, lane);
      else tile_store<float>(acc, y, a, frame, co0, oh0 * W, npx, lane);
    }
  }
}

template <int TH, int W>
int launch_kc_t(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream, DenseQueue** dense) {
  const int groups = (a.c_out + 63) / 64;
  const int nchunks = (a.c_in + 31) / 32;
  const size_t lds = (size_t)2 * kChunkBytes;
  const int64_t tiles = a.n * (int64_t)((a.h_out + TH - 1) / TH);
  const int64_t need = (tiles + kRowsWaves - 1) / kRowsWaves;
  const int per_group = (int)(need < num_cus() ? need : num_cus());
  const int grid = groups * (per_group > 0 ? per_group : 1);
  constexpr auto kern = k_conv_rows_kc<TH, W>;
  const int e = set_lds_limit_once<kern>(kMaxLdsBytes);
  if (e != (int)hipSuccess) return e;
  // (Queue entries hold a run's first pixel of the flattened axis in 31 bits.)
  DenseQueue* dq =
      groups <= kDenseQueueGroups && a.n * (int64_t)a.hw_out < (1ll << 31) ? dense_queue_for(stream) : nullptr;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kRowsWaves), lds, stream, a, a.bits, a.flags, a.x, a.wt, a.bias,
                     a.y, groups, nchunks, in_dtype, out_dtype, dq);
  const int rc = (int)hipGetLastError();
  if (rc == (int)hipSuccess) *dense = dq;
  return rc;
}

}  // namespace

namespace {
int g_num_cus[64] = {0};
}  // namespace

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_num_cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    g_num_cus[dev] = v;
  }
  return g_num_cus[dev];
}

bool rows_kc_applicable(const ConvArgs& a) {
  return a.k == 3 && a.s == 1 && a.p == 1 && a.h_out == a.h_in && a.w_out == a.w_in &&
         (a.w_out == 28 || a.w_out == 14) && a.c_out % 4 == 0 && a.hw_out % 4 == 0 &&
         a.n * (int64_t)a.h_out < (1ll << 30);
}

int launch_conv_rows_kc(const ConvArgs& a, int in_dtype, int out_dtype, hipStream_t stream) {
  DenseQueue* dense = nullptr;
  timing_begin(K_ROWS_KC, stream);
  int rc = a.w_out == 28 ? launch_kc_t<2, 28>(a, in_dtype, out_dtype, stream, &dense)
                         : launch_kc_t<4, 14>(a, in_dtype, out_dtype, stream, &dense);
  timing_end(K_ROWS_KC, stream);
  // The tiles the walk queued for the matrix cores, right after it.
  if (rc == (int)hipSuccess && dense != nullptr) rc = launch_conv_dense_mfma(a, dense, out_dtype, stream);
  return rc;
}

}  // namespace sf
