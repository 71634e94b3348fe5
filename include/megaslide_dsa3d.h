/*
 * megaslide_dsa3d.h -- C ABI of the MI355X (gfx950) 3D Deformable Slide
 * Attention kernels.
 *
 * The library replaces, inside DeformableSlideAttention3D
 * (infinity/video/attention.py:19-273 of the reference):
 *   - the trilinear K/V sampling, local softmax attention and weighted sum
 *     (F.grid_sample x2, matmul, softmax, matmul: attention.py:106-186)
 *     and their autograd backward                    -> msd_dsa3d_fwd / _bwd
 *   - the depthwise Conv3d terms dw_conv (attention.py:58-65, :102) and
 *     offset_net[0:2] = depthwise 3x3x3 conv + GELU (attention.py:71-72, :105)
 *     and their backward                             -> msd_dwconv3d_fwd / _bwd
 * The Linear projections and the 1x1 offset conv stay dense GEMMs in the host
 * framework.
 *
 * Conventions
 *   - Tensors are channel-last: token n = (t*H + h)*W + w, as the reference
 *     flattens video tokens (infinity/video/model.py:206).  q, k, v, out and
 *     their gradients are [B, N, D] with D = num_heads*head_dim and channel
 *     c = head*head_dim + d (attention.py:135-137, :186).
 *   - Offsets are [B, N, C], C = num_heads*kt*kh*kw*3, channel
 *     ((((head*kt + i)*kh + j)*kw + k)*3 + slot): the reference's
 *     offsets.view(B, nh, kt, kh, kw, 3, T, H, W) order (attention.py:109),
 *     unscaled (the kernels multiply by offset_scale, attention.py:106).
 *   - Every pointer is device memory owned by the caller.  No call allocates
 *     or frees device memory, and none keeps a pointer after return (the one
 *     static scratch array of msd_dsa3d_bwd_noalloc comes with the library's
 *     code object).
 *   - `stream` is a hipStream_t (NULL = the null stream).  Work is enqueued;
 *     nothing synchronises the device.
 *   - Return value 0 = success, negative = msd_status; msd_last_error() gives a
 *     thread-local message for the last failure on the calling thread.
 */
#ifndef MEGASLIDE_DSA3D_H
#define MEGASLIDE_DSA3D_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSD_ABI_VERSION 5

typedef enum msd_dtype { MSD_F32 = 0, MSD_BF16 = 1 } msd_dtype;

typedef enum msd_status {
  MSD_OK = 0,
  MSD_ERR_ARG = -1,         /* null pointer, bad size or stride            */
  MSD_ERR_UNSUPPORTED = -2, /* head_dim / kernel / dtype outside the build */
  MSD_ERR_ALIGN = -3,       /* pointer not aligned to its element type     */
  MSD_ERR_WORKSPACE = -4,   /* workspace missing or too small              */
  MSD_ERR_LAUNCH = -5       /* the HIP runtime rejected a launch           */
} msd_status;

/* Shape and options of one attention-core call. */
typedef struct msd_dsa3d_desc {
  int32_t B, T, H, W;          /* batch, latent grid (N = T*H*W)                  */
  int32_t num_heads, head_dim; /* D = num_heads*head_dim                          */
  int32_t kt, kh, kw;          /* window, reference default (3, 7, 7)             */
  int32_t dtype;               /* msd_dtype of q/k/v/offsets/out and their grads  */
  int64_t q_stride;            /* elements between consecutive tokens of q, dq    */
  int64_t k_stride;            /* ... of k, dk                                    */
  int64_t v_stride;            /* ... of v, dv                                    */
  float offset_scale;          /* reference offset_scale (attention.py:106)       */
  float softmax_scale;         /* 1/sqrt(head_dim) in the reference (:176)        */
  int32_t algo;                /* msd_algo: kernel family (MSD_ALGO_AUTO default) */
  /* Attention dropout on the softmax weights (nn.Dropout, attention.py:80,
   * :180).  dropout_p in [0, 1); 0 = off.  The keep mask is drawn from
   * Philox4x32-10 keyed by dropout_seed (see msd_dsa3d_fwd); backward must be
   * called with the same three values as its forward.                        */
  uint32_t dropout_offset;     /* counter word: distinct per call for one seed    */
  uint64_t dropout_seed;       /* generator key                                   */
  float dropout_p;             /* drop probability                                */
  /* Extra keys shared by every query (the reference's extra_kv, attention.py:
   * 160-173): G projected keys and values per sample, appended to each query's
   * kt*kh*kw taps before the softmax.  0 = none; at most 4096 (the tiled
   * kernels take up to 256).                                                 */
  int32_t extra_g;
  /* How msd_dsa3d_bwd sums the dK / dV contributions of different query tiles
   * (msd_accum).  MSD_ACCUM_F32 (0, the default) adds them in fp32, as the
   * reference's grid_sampler_3d_backward does at fp32 grid precision
   * (attention.py:240-273); bf16 dK / dV are rounded once at the end.
   * MSD_ACCUM_F16 (bf16 storage and the tiled kernels only; an error for
   * fp32 storage) adds power-of-two-scaled fp16 pairs instead: about half the
   * atomic traffic, 11 significant bits per running sum, and an fp32 redo of
   * dK / dV when a sum leaves the fp16 range.  The direct kernels always add
   * in fp32.                                                                  */
  int32_t dkv_accum;
} msd_dsa3d_desc;

typedef enum msd_accum { MSD_ACCUM_F32 = 0, MSD_ACCUM_F16 = 1 } msd_accum;

/* Kernel family for the attention core.  AUTO picks the matrix-core tiled
 * kernels when the call qualifies (bf16 or fp32, head_dim 32/64/96/128, <= 160
 * taps, token strides multiples of 8 elements, 16-byte aligned rows) and the
 * direct kernels otherwise.  DIRECT and TILED force one family (TILED fails
 * with MSD_ERR_UNSUPPORTED if not eligible). */
typedef enum msd_algo { MSD_ALGO_AUTO = 0, MSD_ALGO_DIRECT = 1, MSD_ALGO_TILED = 2 } msd_algo;

/* Shape and options of one depthwise-conv call. */
typedef struct msd_dwconv3d_desc {
  int32_t B, T, H, W, C;       /* x and y are [B, T*H*W, C]                       */
  int32_t kt, kh, kw;          /* odd kernel; zero padding kt/2, kh/2, kw/2       */
  int32_t dtype;               /* msd_dtype of x, y, weight, bias and grads       */
  int32_t act;                 /* 0 = none, 1 = exact-erf GELU after the bias     */
} msd_dwconv3d_desc;

/* Version of this header's ABI (MSD_ABI_VERSION). */
int msd_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* msd_last_error(void);

/*
 * Forward of the attention core: replaces attention.py:106-186 (offset scale,
 * base grid + normalised offsets, grid_sample of K and V with border padding
 * and align_corners=False, the extra keys' concatenation, scores / sqrt(hd),
 * softmax, dropout, weighted sum of V).  With dropout_p > 0, tap k (0 <= k <
 * K = kt*kh*kw, in the reference's (i*kh + j)*kw + k order; extra key g is tap
 * K + g) of global token row r = b*N + n and head m is dropped when the first
 * word of Philox4x32-10 (Salmon et al., SC'11) for counter (k, r mod 2^32,
 * (r >> 32) << 16 | m, dropout_offset) and key (dropout_seed mod 2^32,
 * dropout_seed >> 32) is below floor(p * 2^32); kept weights are scaled by
 * 1 / (1 - p) (fp32).
 * extra_k, extra_v: [B, G, D] contiguous, G = desc->extra_g: k_proj and v_proj
 * of the reference's extra_kv; NULL when G = 0.
 * out [B, N, D] (contiguous, token stride D).  lse [B, N, num_heads] fp32
 * receives the log-sum-exp of each query's scores (taps and extra keys) for
 * the backward; it may be NULL when no backward follows.
 */
int msd_dsa3d_fwd(const msd_dsa3d_desc* desc, const void* q, const void* k, const void* v,
                  const void* offsets, const void* extra_k, const void* extra_v, void* out,
                  float* lse, void* stream);

/* Bytes of device workspace msd_dsa3d_bwd needs for `desc`. */
size_t msd_dsa3d_bwd_workspace_size(const msd_dsa3d_desc* desc);

/*
 * Backward of the attention core: the gradients autograd takes through
 * attention.py:106-186 (softmax/matmul backward, grid_sampler_3d_backward for
 * the volumes and the grid, offset normalisation and scale).
 *   out, dout : [B, N, D] contiguous; lse from msd_dsa3d_fwd.
 *   dlse      : optional [B, N, num_heads] fp32 gradient w.r.t. lse (NULL = 0),
 *               for callers that merge extra keys through the log-sum-exp.
 *   dq, dk, dv: written (not accumulated) with the strides of q, k, v.
 *   doffsets  : [B, N, C], gradient w.r.t. the unscaled offsets.
 *   extra_k, extra_v: as for msd_dsa3d_fwd; d_extra_k, d_extra_v: [B, G, D]
 *               contiguous, written; all four NULL when G = 0.
 */
int msd_dsa3d_bwd(const msd_dsa3d_desc* desc, const void* q, const void* k, const void* v,
                  const void* offsets, const void* extra_k, const void* extra_v, const void* out,
                  const void* dout, const float* lse, const float* dlse, void* dq, void* dk,
                  void* dv, void* doffsets, void* d_extra_k, void* d_extra_v, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Largest scratch, in bytes, msd_dsa3d_bwd_noalloc can give a call: what
 * msd_dsa3d_bwd_workspace_size reports for the same descriptor must not exceed
 * it (128 MiB: e.g. B*T*H*W*num_heads*kt*kh*kw up to 16,777,216 taps). */
#define MSD_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

/*
 * msd_dsa3d_bwd without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight training or serving
 * loops, harnesses that forbid hipMalloc).  It has no counterpart in the
 * reference.  Same arguments, results and errors as msd_dsa3d_bwd; its
 * scratch is one static array of MSD_NOALLOC_SCRATCH_BYTES on each GPU that
 * loads this library, held until the process ends, and no call of it
 * allocates or frees memory.  A call whose msd_dsa3d_bwd_workspace_size
 * exceeds MSD_NOALLOC_SCRATCH_BYTES returns MSD_ERR_WORKSPACE.  Every call on
 * one GPU uses that GPU's array and leaves the last call's contents in it:
 * calls that overlap on one GPU (other streams, other host threads) race.
 */
int msd_dsa3d_bwd_noalloc(const msd_dsa3d_desc* desc, const void* q, const void* k,
                          const void* v, const void* offsets, const void* extra_k,
                          const void* extra_v, const void* out, const void* dout,
                          const float* lse, const float* dlse, void* dq, void* dk, void* dv,
                          void* doffsets, void* d_extra_k, void* d_extra_v, void* stream);

/*
 * Depthwise 3-D convolution, channel-last: replaces nn.Conv3d(C, C, k,
 * padding=k//2, groups=C) (attention.py:58-65) and, with act = 1, the
 * offset_net[0:2] pair Conv3d(3, groups=C) + GELU (attention.py:71-72).
 * weight [C, kt*kh*kw] (nn.Conv3d's [C, 1, kt, kh, kw]); bias [C] or NULL.
 * preact (act = 1 only, may be NULL): also receives the GELU input, the
 * tensor nn.GELU's autograd keeps, for msd_dwconv3d_bwd.
 */
int msd_dwconv3d_fwd(const msd_dwconv3d_desc* desc, const void* x, const void* weight,
                     const void* bias, void* y, void* preact, void* stream);

/* Bytes of device workspace msd_dwconv3d_bwd needs for `desc`. */
size_t msd_dwconv3d_bwd_workspace_size(const msd_dwconv3d_desc* desc);

/*
 * Backward of msd_dwconv3d_fwd (conv3d input/weight backward, GELU backward).
 * With act = 1 the GELU gradient uses preact, the forward's saved GELU input,
 * or, when preact is NULL, recomputes it (one more convolution).  dx,
 * dweight, dbias may each be NULL when not wanted; dx is written, not
 * accumulated.
 */
int msd_dwconv3d_bwd(const msd_dwconv3d_desc* desc, const void* x, const void* weight,
                     const void* bias, const void* preact, const void* dy, void* dx,
                     void* dweight, void* dbias, void* workspace, size_t workspace_bytes,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEGASLIDE_DSA3D_H */
