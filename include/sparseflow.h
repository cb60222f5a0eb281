/*
 * sparseflow.h -- C ABI of libsparseflow_hip.so, the MI355X (gfx950) kernels
 * behind the SparseFlow spike-sparse convolution path.
 *
 * Every entry point takes raw device pointers, plain sizes and a hipStream_t
 * passed as `void*` (NULL = the null stream).  Nothing here allocates device
 * memory, synchronises the host, or depends on torch types.  All functions
 * return an sf_status; on failure sf_last_error() describes the cause.
 *
 * Data layouts (all row-major, C-contiguous):
 *   x       [n, c_in, h_in, w_in]          NCHW activations (f32 / f16 / bf16)
 *   bits    [n, h_in*w_in, cwp] uint32     channel-packed spike bitmap: bit
 *                                          (c & 31) of word (c >> 5) of pixel
 *                                          p is 1 iff f16(|x[n,c,p]|) > f16(thr)
 *                                          cwp = sf_bitmap_words_per_pixel(c_in)
 *           (sf_bitmap_layout: the same words may also be laid out as word
 *           planes [n, cwp, h_in*w_in], see the *_layout entry points)
 *   flags   [n, ceil(h*w / chunk)] uint32  1 where a pixel chunk holds a value
 *                                          outside {0, 1} (chunk is chosen by
 *                                          the library from the shape)
 *   wt      [c_in*k*k, c_out] f32          weights, tap-major: row
 *                                          (ci*k + kh)*k + kw holds w[:,ci,kh,kw]
 *   y       [n, c_out, h_out, w_out]       NCHW output, dtype = desc.out_dtype
 *
 * Determinism: every output element is produced by exactly one lane of one
 * wavefront, summing bias first and then its active taps in an order fixed by
 * the shape (no atomics).  Repeated calls on the same inputs are
 * bit-identical.
 */
#ifndef SPARSEFLOW_H
#define SPARSEFLOW_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum sf_status {
  SF_OK = 0,
  SF_ERR_INVALID = 1,      /* bad pointer, size or parameter */
  SF_ERR_UNSUPPORTED = 2,  /* shape/pattern the kernels do not implement;
                              callers fall back to a dense conv */
  SF_ERR_WORKSPACE = 3,    /* workspace smaller than sf_*_workspace_size */
  SF_ERR_HIP = 4           /* HIP runtime error (launch / event) */
} sf_status;

typedef enum sf_dtype { SF_F32 = 0, SF_F16 = 1, SF_BF16 = 2 } sf_dtype;

/* Shape of one 2-D convolution over n frames (n = N, or T*N for 5-D input). */
typedef struct sf_conv_desc {
  int64_t n;
  int32_t c_in, h_in, w_in;
  int32_t c_out, h_out, w_out;
  int32_t kernel, stride, pad;   /* supported: (3,1,1) (3,2,1) (1,1,0) (1,2,0) */
  int32_t in_dtype, out_dtype;   /* sf_dtype */
} sf_conv_desc;

/* Order of a spike bitmap's words.  PIXEL_MAJOR: [n, h*w, cwp] (the
 * cwp words of a pixel together; sf_prescan_pack's layout).  PLANES:
 * [n, cwp, h*w] (word w of every pixel of a frame together), which the 3x3
 * pixel-tile and row kernels read one run per load.  With cwp == 1 the two
 * coincide. */
typedef enum sf_bitmap_layout { SF_BITMAP_PIXEL_MAJOR = 0, SF_BITMAP_PLANES = 1 } sf_bitmap_layout;

/* Multi-step LIF neuron (spikingjelly LIFNode semantics). */
typedef struct sf_lif_params {
  float tau;
  float v_threshold;
  float v_reset;        /* used when hard_reset != 0; 0.0 enters the decay otherwise */
  int32_t hard_reset;   /* 1: v <- v_reset on spike; 0: v <- v - v_threshold */
  int32_t decay_input;  /* 1: H = V + (I - (V - Vr))/tau; 0: H = V - (V - Vr)/tau + I */
} sf_lif_params;

/* ---- library / host utilities (no GPU needed) --------------------------- */

/* Library ABI version (major*10000 + minor*100 + patch). */
int sf_version(void);

/* Message for the last failing call on this host thread ("" if none). */
const char* sf_last_error(void);

/* Smallest float c >= 0 such that f16(|v|) > f16(threshold) <=> |v| >= c for
 * every non-NaN float v.  Restates the prescan comparison of an fp16 tensor
 * against a Python float (Kernels/_prescan_common.py:188, `tile_max > thr`). */
float sf_activity_cutoff(float threshold);

/* uint32 words per pixel in the spike bitmap: next power of two of
 * ceil(c/32), at least 1. */
int sf_bitmap_words_per_pixel(int32_t c);

/* Pixels per non-binary flag chunk for n frames of c x h x w (flag word
 * f*cpf + j covers pixels [j*chunk, (j+1)*chunk) of frame f). */
int32_t sf_prescan_chunk_pixels(int64_t n, int32_t c, int32_t h, int32_t w);

/* Bytes of the bitmap and the chunk-flag array for n frames of c x h x w. */
size_t sf_prescan_bitmap_bytes(int64_t n, int32_t c, int32_t h, int32_t w);
size_t sf_prescan_flags_bytes(int64_t n, int32_t c, int32_t h, int32_t w);

/* Workspace for sf_conv2d_forward (bitmap + flags over desc->n frames, in
 * 256-byte aligned sections). */
size_t sf_conv2d_workspace_size(const sf_conv_desc* desc);

/* Workspace for sf_conv_lif_forward over T steps of desc->n samples. */
size_t sf_conv_lif_workspace_size(const sf_conv_desc* desc, int32_t T);

/* ---- Stage 1: prescan ---------------------------------------------------- */

/* Stage 1a.  Stream x once (128-bit loads) and write the channel-packed
 * spike bitmap plus per-chunk non-binary flags.
 * Replaces the fp16 cast + group amax of the reference prescan
 * (Kernels/conv2d.py:986, Kernels/_prescan_common.py:32-45,167). */
int sf_prescan_pack(const void* x, int32_t dtype, int64_t n, int32_t c,
                    int32_t h, int32_t w, float threshold, uint32_t* bits,
                    uint32_t* flags, void* stream);

/* Stage 1b.  For every output tile (n, gh, gw) of tile_h x tile_w output
 * pixels, OR the bitmap over the tile's receptive field (kernel, stride,
 * pad) and emit, each output optional (NULL skips it):
 *   ch_mask    [tiles, cwp] uint32  active-channel mask (group size 1)
 *   ch_count   [tiles]      int32   popcount of ch_mask
 *   ch_list    [tiles, c]   int32   ascending active channel ids, compacted
 *                                   through an LDS prefix sum; entries past
 *                                   ch_count are left unwritten
 *   ag_mask    [tiles]      int32   bit g = group g (group_size channels)
 *                                   active; the reference's ag_mask
 *   tile_class [tiles]      int32   0 zero / 1 sparse / 2 all groups active
 * Tile index = (n*GH + gh)*GW + gw, GH = ceil(h_out/tile_h).
 * Replaces _build_rf_prescan_metadata_impl / _prescan_2d_impl /
 * _classify_tiles (Kernels/_prescan_common.py:231-275,153-189,57-109). */
int sf_prescan_tiles(const uint32_t* bits, int64_t n, int32_t c, int32_t h_in,
                     int32_t w_in, int32_t h_out, int32_t w_out, int32_t kernel,
                     int32_t stride, int32_t pad, int32_t tile_h, int32_t tile_w,
                     int32_t group_size, uint32_t* ch_mask, int32_t* ch_count,
                     int32_t* ch_list, int32_t* ag_mask, int32_t* tile_class,
                     void* stream);

/* ---- Stage 2: sparse convolution ----------------------------------------- */

/* Sparse conv over a bitmap produced by sf_prescan_pack for the same x.
 * Binary chunks add weight rows; chunks flagged non-binary read x and FMA.
 * bias may be NULL.  Kernel choice, by shape: 3x3 with c_in * 9 <= 32 and
 * fp32 input (an image stem) runs the matrix-core kernel ("conv_mfma"); 3x3
 * stride 1 with c_in <= 64 on frames of width 32 runs the row-band kernel
 * ("conv_rows"); 3x3 stride 1 on frames of width 28 or 14 with c_out and h*w
 * multiples of 4 runs the K-chunked row kernel ("conv_rows_kc") unless the
 * pixel-tile kernel keeps its weights resident; other 3x3 (stride 1 or 2)
 * with c_out a multiple of 4 runs the pixel-tile kernel ("conv_px3"); 1x1
 * stride 1 with c_out a multiple of 4 runs the flat-tile kernel
 * ("conv_flat"); every other supported shape runs the gather kernel
 * ("conv_gather").  Replaces sparse_conv3x3s1/s2 and conv1x1 NHWC kernels
 * (Kernels/conv2d.py:237-361,564-886) and the persistent fused 1x1 kernel
 * (Kernels/conv2d.py:364-460). */
int sf_conv2d_sparse(const sf_conv_desc* desc, const uint32_t* bits,
                     const uint32_t* flags, const void* x, const float* wt,
                     const float* bias, void* y, void* stream);

/* The bitmap layout that the Stage-2 kernel sf_conv2d_sparse picks for desc
 * reads fastest: SF_BITMAP_PLANES for the 3x3 pixel-tile ("conv_px3") and
 * K-chunked row ("conv_rows_kc") kernels, SF_BITMAP_PIXEL_MAJOR otherwise.
 * A neuron layer that hands its spike map to this convolution writes it in
 * that layout (sf_lif_multistep_layout, sf_conv1x1_lif_sparse_layout).
 * Returns a negative sf_status for an invalid desc. */
int sf_conv2d_bitmap_layout(const sf_conv_desc* desc);

/* sf_conv2d_sparse on a bitmap in the given sf_bitmap_layout.  PLANES is
 * taken where sf_conv2d_bitmap_layout(desc) is PLANES or cwp == 1, else
 * SF_ERR_UNSUPPORTED (the caller prescans x instead).  Same kernels and
 * results as sf_conv2d_sparse, bit for bit.  Same reference interface as
 * sf_conv2d_sparse (the handed map itself has no counterpart there). */
int sf_conv2d_sparse_layout(const sf_conv_desc* desc, const uint32_t* bits,
                            int32_t layout, const uint32_t* flags,
                            const void* x, const float* wt, const float* bias,
                            void* y, void* stream);

/* Stage 1a + Stage 2 in one call; the bitmap lives in `workspace`.  3x3
 * stride-1 layers with c_in <= 64 on 32-wide frames (other than an image
 * stem) run as one launch with the prescan fused into the conv
 * ("conv_rows_fused"; the workspace is then unused).  The workspace's
 * contents are private to the call: when Stage 2 is the pixel-tile kernel
 * the bitmap is written as word planes [n, cwp, h_in*w_in] instead of
 * sf_prescan_pack's [n, h_in*w_in, cwp] (same words, same size).
 * Replaces sparse_conv2d_forward's device work (Kernels/conv2d.py:893-1178). */
int sf_conv2d_forward(const sf_conv_desc* desc, const void* x, const float* wt,
                      const float* bias, float threshold, void* workspace,
                      size_t workspace_bytes, void* y, void* stream);

/* Bytes of the library-owned scratch area behind sf_conv2d_forward_noalloc
 * (one per GPU, held from the library's load on that GPU to process exit). */
#define SF_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* sf_conv2d_forward without a workspace argument: the bitmap and flags live
 * in the library's scratch area, so the call allocates nothing (no hipMalloc,
 * no allocating library routine).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  Limit:
 * sf_conv2d_workspace_size(desc) <= SF_NOALLOC_SCRATCH_BYTES, else
 * SF_ERR_WORKSPACE before any launch (e.g. 512 frames of 64 x 56 x 56 need
 * 12.9 MB).  Every call on one GPU uses that GPU's single scratch area:
 * calls that overlap on one GPU (several streams or host threads) race;
 * calls ordered on one stream do not.  Results equal sf_conv2d_forward's bit
 * for bit (same kernels).  The first call on each GPU looks up the device
 * addresses of the library's scratch and queue arrays (which may load the
 * library's code objects on that GPU): make that first call outside graph
 * capture; every later call on the GPU only launches kernels. */
int sf_conv2d_forward_noalloc(const sf_conv_desc* desc, const void* x,
                              const float* wt, const float* bias,
                              float threshold, void* y, void* stream);

/* Fused sparse conv + multi-step LIF.  x is [T, N, c_in, h, w] (desc->n = N),
 * spikes [T, N, c_out, h_out, w_out] in desc->out_dtype, v_out [N, c_out,
 * h_out, w_out] f32 = membrane after step T.  v_init (f32, same shape as
 * v_out) may be NULL for V_0 = 0.  The membrane stays in registers across the
 * T steps.  Replaces fused_bm_conv3x3_lif_8x8/8x16 + the module's T loop
 * (Kernels/fused_conv_lif.py:63-303,310-484; Ops/sparse_fused_conv_lif.py:
 * 184-225,271-293). */
int sf_conv_lif_forward(const sf_conv_desc* desc, int32_t T, const void* x,
                        const float* wt, const float* bias,
                        const sf_lif_params* lif, float threshold,
                        const float* v_init, void* spikes, float* v_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Fused 1x1 stride-1 conv + multi-step LIF on a prescanned (or handed) spike
 * map of the input: x [T, N, c_in, h, w] (desc->n = N) with its bitmap and
 * flags over the T*N frames; x2 (optional, [T, N, c_out, h, w], in_dtype) is
 * added into every step's current (a residual: LIF(conv(x) + x2)); spikes
 * [T, N, c_out, h, w] in desc->out_dtype, v_out [N, c_out, h, w] f32 after
 * step T, v_init as sf_conv_lif_forward.  out_bits / out_flags (both or
 * neither) receive the spikes' spike map in the layout sf_prescan_pack
 * produces for the T*N output frames (flags all zero), for the next sparse
 * convolution.  c_out % 4 == 0.  The membrane is carried in the
 * accumulators across the T steps (the update of sf_conv_lif_forward, equal
 * to an unfused conv + LIF up to rounding).  Extends the reference's fused
 * conv-LIF (Kernels/fused_conv_lif.py:310-484, 3x3 only there) to the 1x1
 * convolutions of its bottleneck models, with the residual add and the
 * spike map, which have no counterpart in the reference. */
int sf_conv1x1_lif_sparse(const sf_conv_desc* desc, int32_t T,
                          const uint32_t* bits, const uint32_t* flags,
                          const void* x, const float* wt, const float* bias,
                          const void* x2, const sf_lif_params* lif,
                          const float* v_init, void* spikes, float* v_out,
                          uint32_t* out_bits, uint32_t* out_flags, void* stream);

/* sf_conv1x1_lif_sparse with a binary residual (values 0 / 1 only, e.g. the
 * spikes entering a bottleneck) given by its spike map instead of its
 * values: res_bits in the layout of out_bits
 * (sf_bitmap_words_per_pixel(c_out) words per pixel of the T*n frames).  The
 * results equal those of sf_conv1x1_lif_sparse on the residual's values; the
 * residual costs 1/32 of its fp32 bytes.  Same reference interface as
 * sf_conv1x1_lif_sparse (the identity add of the reference models'
 * bottlenecks, Benchmark/bench_4test.py:166-197). */
int sf_conv1x1_lif_sparse_binres(const sf_conv_desc* desc, int32_t T,
                                 const uint32_t* bits, const uint32_t* flags,
                                 const void* x, const float* wt, const float* bias,
                                 const uint32_t* res_bits, const sf_lif_params* lif,
                                 const float* v_init, void* spikes, float* v_out,
                                 uint32_t* out_bits, uint32_t* out_flags, void* stream);

/* sf_conv1x1_lif_sparse with the output spike map written in out_layout
 * (sf_bitmap_layout); the input bitmap is pixel-major as there.  Same
 * reference interface as sf_conv1x1_lif_sparse. */
int sf_conv1x1_lif_sparse_layout(const sf_conv_desc* desc, int32_t T,
                                 const uint32_t* bits, const uint32_t* flags,
                                 const void* x, const float* wt, const float* bias,
                                 const void* x2, const sf_lif_params* lif,
                                 const float* v_init, void* spikes, float* v_out,
                                 uint32_t* out_bits, uint32_t* out_flags,
                                 int32_t out_layout, void* stream);

/* ---- spiking neuron -------------------------------------------------------- */

/* Multi-step LIF over T steps of n x c x hw neurons: x [T, n, c, hw] input
 * currents (in_dtype), plus x2 (same layout and dtype, may be NULL) summed
 * into the current and rounded once -- a residual add fused into the neuron
 * layer; spikes [T, n, c, hw] in out_dtype (in_dtype or f32); v_out [n, c, hw]
 * f32 = membrane after step T.  v_init (f32, same layout as v_out) may be
 * NULL for V_0 = v_reset (hard reset) or 0 (soft reset).  Same update as
 * sf_conv_lif_forward, computed operation by operation without fused
 * multiply-adds.  When bits and flags are given the spike map of the T*n
 * output frames is written in the layout sf_prescan_pack produces for them
 * (sf_prescan_bitmap_bytes / sf_prescan_flags_bytes(T*n, c, 1, hw) bytes;
 * flags all zero), so sf_conv2d_sparse can consume the spikes without a
 * prescan.  Replaces spikingjelly's multi-step LIFNode used between the
 * convolutions of the reference's spiking models (Benchmark/bench_4test.py:
 * 166-197; update rule as restated in Ops/sparse_fused_conv_lif.py:283-292);
 * the spike map output has no counterpart in the reference. */
int sf_lif_multistep(const void* x, const void* x2, int32_t in_dtype, int32_t T,
                     int64_t n, int32_t c, int64_t hw, const sf_lif_params* lif,
                     const float* v_init, void* spikes, int32_t out_dtype,
                     float* v_out, uint32_t* bits, uint32_t* flags, void* stream);

/* sf_lif_multistep with the spike map written in bits_layout
 * (sf_bitmap_layout).  Same reference interface as sf_lif_multistep. */
int sf_lif_multistep_layout(const void* x, const void* x2, int32_t in_dtype,
                            int32_t T, int64_t n, int32_t c, int64_t hw,
                            const sf_lif_params* lif, const float* v_init,
                            void* spikes, int32_t out_dtype, float* v_out,
                            uint32_t* bits, uint32_t* flags, int32_t bits_layout,
                            void* stream);

/* Max pooling (kernel k, stride, padding <= k/2, floor mode) of n frames of a
 * binary spike tensor [c, h_in, w_in] given only by its spike map `bits`
 * (the pixel-major words sf_prescan_pack and sf_lif_multistep write): the max
 * of 0 / 1 values over a window is the OR of the window's words.  Writes the
 * pooled spikes y [n, c, h_out, w_out] (0 / 1 in out_dtype) and their spike
 * map out_bits in the same layout (its flags are all zero: the caller hands
 * zeroed flags of sf_prescan_flags_bytes(n, c, h_out, w_out) bytes with it).
 * c <= 256.  Replaces, for spike inputs, the nn.MaxPool2d after the stem
 * neuron of the reference's spiking ResNets (F.max_pool2d on the dense
 * spikes); the spike-map form has no counterpart in the reference. */
int sf_spike_maxpool2d(const uint32_t* bits, int64_t n, int32_t c, int32_t h_in,
                       int32_t w_in, int32_t k, int32_t stride, int32_t padding,
                       void* y, int32_t out_dtype, uint32_t* out_bits, void* stream);

/* ---- sparse linear ------------------------------------------------------------ */

/* y[m, c_out] = x[m, k] @ wt[k, c_out] + bias for a spike-sparse row-major x
 * (any leading shape flattened to m rows; wt = weight transposed, f32).
 * Replaces the reference's sparse_linear_forward (Kernels/linear.py:460-778:
 * grouped prescan + tile classification + sparse_linear_grouped_kernel) for
 * the Linear layers of its spiking transformers (Ops/sparse_linear.py:68-890).
 *
 * Stage 1 (sf_linear_prescan): one bit per element, bit j of word w of row r
 * = f16(|x[r, 32w + j]|) > f16(threshold) (the test sf_prescan_pack applies),
 * sf_linear_bitmap_bytes(m, k) bytes; one non-binary flag word per 16 rows
 * (sf_linear_flags_bytes(m)), non-zero when a row of the chunk holds a value
 * other than 0 and 1.  Stage 2 (sf_linear_sparse): each output row sums the
 * weight rows of its active elements (times the element where the chunk is
 * flagged) in increasing k; deterministic.  c_out must be a multiple of 4;
 * out_dtype = in_dtype or f32; m < 2^30.  sf_linear_forward runs both with
 * the bitmap in `workspace` (sf_linear_workspace_size(m, k) bytes). */
size_t sf_linear_bitmap_bytes(int64_t m, int32_t k);
size_t sf_linear_flags_bytes(int64_t m);
size_t sf_linear_workspace_size(int64_t m, int32_t k);
int sf_linear_prescan(const void* x, int32_t dtype, int64_t m, int32_t k,
                      float threshold, uint32_t* bits, uint32_t* flags,
                      void* stream);
int sf_linear_sparse(const uint32_t* bits, const uint32_t* flags, const void* x,
                     int32_t in_dtype, int64_t m, int32_t k, const float* wt,
                     const float* bias, int32_t c_out, void* y,
                     int32_t out_dtype, void* stream);
int sf_linear_forward(const void* x, int32_t in_dtype, int64_t m, int32_t k,
                      const float* wt, const float* bias, int32_t c_out,
                      float threshold, void* workspace, size_t workspace_bytes,
                      void* y, int32_t out_dtype, void* stream);

/* The same product on the matrix cores, for inputs whose every 32-wide K
 * slice is live in some row of a 128-row tile (transformer densities): W
 * given as bf16 hi and lo parts (w_hi = bf16(W), w_lo = bf16(W - w_hi)),
 * [c_out][kp] with kp = k rounded up to a multiple of 32 (zero padded),
 * 16-byte aligned; y = x @ (w_hi + w_lo)^T + bias, with x split the same way
 * in the kernel (exact for spikes and small integers; ~16 bits otherwise);
 * elements with f16(|x|) <= f16(threshold) count as zero.  Every product is
 * computed (dense tiles, the reference's all-groups-active case).  No
 * prescan, no workspace.  k <= 8192; c_out a multiple of 4 (the output is
 * stored as 16-byte row pieces). */
int sf_linear_mfma(const void* x, int32_t in_dtype, int64_t m, int32_t k,
                   const uint16_t* w_hi, const uint16_t* w_lo, int32_t kp,
                   const float* bias, int32_t c_out, float threshold, void* y,
                   int32_t out_dtype, void* stream);

/* sf_linear_mfma over sf_linear_prescan's row bitmap and flags (computed
 * from the same x and threshold): a 128-row block whose flag words are all
 * zero (spikes, the transformer case) takes its A operand from the bitmap
 * (4 bytes of x per row per 32-wide K step instead of 128), a flagged block
 * reads x; same products, same results as sf_linear_mfma to rounding
 * (bit-identical for binary rows).  Replaces the reference's
 * sparse_linear_grouped_kernel (Kernels/linear.py:360-457) after its
 * group-bitmask metadata (Kernels/linear.py:110-357);
 * m * words_per_row * 4 < 2^31; c_out a multiple of 4. */
int sf_linear_mfma_bits(const uint32_t* bits, const uint32_t* flags,
                        const void* x, int32_t in_dtype, int64_t m, int32_t k,
                        const uint16_t* w_hi, const uint16_t* w_lo, int32_t kp,
                        const float* bias, int32_t c_out, float threshold,
                        void* y, int32_t out_dtype, void* stream);

/* ---- sparse batched matmul -------------------------------------------------- */

/* c[b] = alpha * (a[b] @ B[b]) for b < batches: a [batches, m, k] contiguous and
 * spike-sparse, B read at B[b*b_stride_batch + kk*b_stride_k + j*b_stride_n]
 * (elements; a transposed view such as K^T needs no copy), c [batches, m, n]
 * contiguous in out_dtype (in_dtype or f32).  a and B share in_dtype.
 * Elements of a with f16(|a|) <= f16(threshold) are skipped; the rest are
 * summed in f32 in increasing k (deterministic).  Supported while
 * sf_bmm_supported(k, n) (k <= 252).  Replaces the reference's
 * sparse_bmm_forward (Kernels/bmm.py:195-361) used by its sparse attention
 * (Kernels/attention.py:27-121, Ops/sparse_bmm.py:22-131). */
int sf_bmm_supported(int32_t k, int32_t n);
/* The same product on the matrix cores, for the attention shapes (rows of a
 * dense enough that every 32-wide K slice of a 16-row tile is live): B and
 * each 16-row tile of a split into bf16 hi + lo parts (~16 bits of both
 * operands), all products computed.  Same arguments and bar as
 * sf_bmm_sparse; supported while sf_bmm_mfma_supported(k, n) (k <= 256 and
 * roundup(n, 16) * roundup(k, 32) <= 16384). */
int sf_bmm_mfma_supported(int32_t k, int32_t n);
int sf_bmm_mfma(const void* a, const void* b, int32_t in_dtype, int64_t batches,
                int32_t m, int32_t k, int32_t n, int64_t b_stride_batch,
                int64_t b_stride_k, int64_t b_stride_n, float threshold,
                float alpha, void* c, int32_t out_dtype, void* stream);
int sf_bmm_sparse(const void* a, const void* b, int32_t in_dtype, int64_t batches,
                  int32_t m, int32_t k, int32_t n, int64_t b_stride_batch,
                  int64_t b_stride_k, int64_t b_stride_n, float threshold,
                  float alpha, void* c, int32_t out_dtype, void* stream);

/* ---- fused spike attention ------------------------------------------------ */

/* Softmax-free attention core of spiking transformers, per frame tb and head:
 * y[tb, m, h, :] = scale * sum_d q[tb, m, h, d] * (k^T v)[tb, h, d, :], which
 * equals (q @ k^T * scale) @ v of the reference's two attention stages
 * (Kernels/attention.py:27-121; Models/spikformer_github.py:141-146) without
 * materialising the s x s scores.  Element (tb, m, h, d) of q, k and v is at
 * tb*qkv_strides[0] + m*qkv_strides[1] + h*qkv_strides[2] + d, of y at the
 * same form with y_strides (elements; d contiguous).  q elements with
 * f16(|q|) <= f16(threshold) count as zero.  head_dim d in {16, 32, 64};
 * supported while sf_spike_attention_supported(s, d).  No counterpart entry
 * point in the reference (it runs the two stages as separate bmm calls). */
int sf_spike_attention_supported(int32_t s, int32_t d);
int sf_spike_attention(const void* q, const void* k, const void* v,
                       int32_t in_dtype, int64_t tb, int32_t s, int32_t h,
                       int32_t d, const int64_t* qkv_strides, float scale,
                       float threshold, void* y, const int64_t* y_strides,
                       int32_t out_dtype, void* stream);

/* ---- per-kernel timing (bench instrumentation) --------------------------- */

/* When enabled, every kernel launched by the library is bracketed by a
 * hipEvent pair on its stream.  sf_timing_collect synchronises those events
 * and accumulates per-kernel totals; sf_timing_query reads them by name
 * ("prescan_pack", "prescan_tiles", "conv_gather", "conv_lif", "conv_rows",
 * "conv_rows_kc", "conv_flat", "conv_px3", "conv_lif_px3", "lif_multistep",
 * "prescan_rows", "linear_flat", "bmm_sparse", "spike_attention",
 * "linear_mfma", "bmm_mfma", "conv_lif_flat", "conv_mfma", "conv_rows_fused",
 * "conv_dense_mfma").
 * Returns the
 * number of launches recorded for that kernel. */
int sf_timing_enable(int32_t enable);
int sf_timing_collect(void);
int64_t sf_timing_query(const char* kernel, double* total_ms);
void sf_timing_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEFLOW_H */
