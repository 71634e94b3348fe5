// C ABI entry points: argument validation, error reporting, dispatch to the
// kernel launchers.  Declarations and conventions: include/megaslide_dsa3d.h.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "common.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err[0] = '\0';
    return MSD_OK;
  }
  return fail(MSD_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

size_t elem_bytes(int32_t dtype) { return dtype == MSD_BF16 ? 2 : 4; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_dsa(const msd_dsa3d_desc* d) {
  if (d == nullptr) return fail(MSD_ERR_ARG, "dsa3d: desc is NULL");
  if (d->B < 0 || d->T < 1 || d->H < 1 || d->W < 1)
    return fail(MSD_ERR_ARG, "dsa3d: bad shape B=%d T=%d H=%d W=%d", d->B, d->T, d->H, d->W);
  if (d->num_heads < 1 || d->head_dim < 1)
    return fail(MSD_ERR_ARG, "dsa3d: bad heads num_heads=%d head_dim=%d", d->num_heads,
                d->head_dim);
  if (d->head_dim > msd::dsa3d_max_head_dim())
    return fail(MSD_ERR_UNSUPPORTED, "dsa3d: head_dim=%d above the supported %d", d->head_dim,
                msd::dsa3d_max_head_dim());
  if (d->kt < 1 || d->kh < 1 || d->kw < 1)
    return fail(MSD_ERR_ARG, "dsa3d: bad window (%d, %d, %d)", d->kt, d->kh, d->kw);
  if (d->dtype != MSD_F32 && d->dtype != MSD_BF16)
    return fail(MSD_ERR_UNSUPPORTED, "dsa3d: dtype %d not supported", d->dtype);
  if (d->algo < MSD_ALGO_AUTO || d->algo > MSD_ALGO_TILED)
    return fail(MSD_ERR_ARG, "dsa3d: bad algo %d", d->algo);
  if (d->extra_g < 0 || d->extra_g > 4096)
    return fail(MSD_ERR_ARG, "dsa3d: extra_g %d outside [0, 4096]", d->extra_g);
  if (d->dkv_accum != MSD_ACCUM_F32 && d->dkv_accum != MSD_ACCUM_F16)
    return fail(MSD_ERR_ARG, "dsa3d: bad dkv_accum %d", d->dkv_accum);
  if (d->dkv_accum == MSD_ACCUM_F16 && d->dtype != MSD_BF16)
    return fail(MSD_ERR_ARG, "dsa3d: dkv_accum MSD_ACCUM_F16 needs bf16 storage");
  if (!(d->dropout_p >= 0.0f && d->dropout_p < 1.0f))
    return fail(MSD_ERR_ARG, "dsa3d: dropout_p %g outside [0, 1)", static_cast<double>(d->dropout_p));
  const int64_t D = static_cast<int64_t>(d->num_heads) * d->head_dim;
  if (d->q_stride < D || d->k_stride < D || d->v_stride < D)
    return fail(MSD_ERR_ARG, "dsa3d: token strides (%lld, %lld, %lld) below D=%lld",
                (long long)d->q_stride, (long long)d->k_stride, (long long)d->v_stride,
                (long long)D);
  const int64_t N = static_cast<int64_t>(d->T) * d->H * d->W;
  const int64_t C = static_cast<int64_t>(d->num_heads) * d->kt * d->kh * d->kw * 3;
  if (C > (int64_t(1) << 30) || N > (int64_t(1) << 40) || static_cast<int64_t>(d->B) * N > (int64_t(1) << 40))
    return fail(MSD_ERR_ARG, "dsa3d: sizes out of range");
  return MSD_OK;
}

int check_ptrs(const char* what, size_t align, std::initializer_list<const void*> ps) {
  int i = 0;
  for (const void* p : ps) {
    if (p == nullptr) return fail(MSD_ERR_ARG, "%s: pointer argument %d is NULL", what, i);
    if (!aligned(p, align))
      return fail(MSD_ERR_ALIGN, "%s: pointer argument %d not %zu-byte aligned", what, i, align);
    ++i;
  }
  return MSD_OK;
}

int check_conv(const msd_dwconv3d_desc* d) {
  if (d == nullptr) return fail(MSD_ERR_ARG, "dwconv3d: desc is NULL");
  if (d->B < 0 || d->T < 1 || d->H < 1 || d->W < 1 || d->C < 1)
    return fail(MSD_ERR_ARG, "dwconv3d: bad shape B=%d T=%d H=%d W=%d C=%d", d->B, d->T, d->H,
                d->W, d->C);
  if (d->kt < 1 || d->kh < 1 || d->kw < 1 || !(d->kt & 1) || !(d->kh & 1) || !(d->kw & 1))
    return fail(MSD_ERR_UNSUPPORTED, "dwconv3d: kernel (%d, %d, %d) must be odd and >= 1", d->kt,
                d->kh, d->kw);
  if (d->dtype != MSD_F32 && d->dtype != MSD_BF16)
    return fail(MSD_ERR_UNSUPPORTED, "dwconv3d: dtype %d not supported", d->dtype);
  if (d->act != 0 && d->act != 1) return fail(MSD_ERR_UNSUPPORTED, "dwconv3d: act %d", d->act);
  return MSD_OK;
}

// Scratch of msd_dsa3d_bwd_noalloc: one array on every GPU that loads the
// library, held until the process ends.  Host code never passes the array's
// name (a host-side stand-in) to a kernel: it uses the per-device address that
// hipGetSymbolAddress returns.  Calls that overlap on one GPU share it and race.
constexpr size_t kNoAllocScratchBytes = MSD_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device
// with that device current.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(MSD_ERR_LAUNCH, "dsa3d_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MSD_ERR_UNSUPPORTED, "dsa3d_bwd_noalloc: device %d beyond the %d supported", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(MSD_ERR_LAUNCH, "dsa3d_bwd_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MSD_OK;
}

int dsa3d_bwd_impl(const msd_dsa3d_desc* desc, const void* q, const void* k, const void* v,
                   const void* offsets, const void* ek, const void* ev, const void* out,
                   const void* dout, const float* lse, const float* dlse, void* dq, void* dk,
                   void* dv, void* doffsets, void* dek, void* dev, void* workspace,
                   size_t workspace_bytes, void* stream, bool noalloc) {
  int rc = check_dsa(desc);
  if (rc != MSD_OK) return rc;
  rc = check_ptrs("dsa3d_bwd", elem_bytes(desc->dtype),
                  {q, k, v, offsets, out, dout, dq, dk, dv, doffsets});
  if (rc != MSD_OK) return rc;
  if (desc->extra_g > 0) {
    rc = check_ptrs("dsa3d_bwd(extra_k, extra_v, d_extra_k, d_extra_v)", 16, {ek, ev, dek, dev});
    if (rc != MSD_OK) return rc;
  }
  rc = check_ptrs("dsa3d_bwd(lse)", 4, {lse});
  if (rc != MSD_OK) return rc;
  if (dlse != nullptr && !aligned(dlse, 4)) return fail(MSD_ERR_ALIGN, "dsa3d_bwd: dlse misaligned");
  if (desc->B == 0) return MSD_OK;
  const size_t need = msd::dsa3d_bwd_ws_bytes(*desc);
  if (noalloc) {
    if (need > kNoAllocScratchBytes)
      return fail(MSD_ERR_WORKSPACE,
                  "dsa3d_bwd_noalloc: the call needs %zu bytes of scratch, above the %zu-byte "
                  "maximum of the no-allocation entry point (use msd_dsa3d_bwd with a workspace)",
                  need, kNoAllocScratchBytes);
    rc = scratch_address(&workspace);
    if (rc != MSD_OK) return rc;
    workspace_bytes = kNoAllocScratchBytes;
  }
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 16)))
    return fail(MSD_ERR_WORKSPACE, "dsa3d_bwd: workspace of %zu bytes (16-aligned) needed, got %zu",
                need, workspace == nullptr ? size_t(0) : workspace_bytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // the tiled backward also writes dq with 16-byte rows and reads out/dout rows of D
  const bool tiled_ok = msd::dsa3d_tiled_supported(*desc, q, k, v) &&
                        msd::dsa3d_tiled_supported(*desc, dq, dk, dv);
  if (desc->algo == MSD_ALGO_TILED && !tiled_ok)
    return fail(MSD_ERR_UNSUPPORTED,
                "dsa3d_bwd: tiled kernels need bf16 or fp32, head_dim 32, 64, 96 or 128, <= 160 taps, "
                "<= 256 extra keys and 16-byte aligned rows");
  if (tiled_ok && desc->algo != MSD_ALGO_DIRECT)
    return launch_status(msd::launch_dsa3d_bwd_tiled(*desc, q, k, v, offsets, ek, ev, out, dout,
                                                     lse, dlse, dq, dk, dv, doffsets, dek, dev,
                                                     workspace, s),
                         "dsa3d_bwd");
  return launch_status(msd::launch_dsa3d_bwd_direct(*desc, q, k, v, offsets, ek, ev, out, dout,
                                                    lse, dlse, dq, dk, dv, doffsets, dek, dev,
                                                    workspace, s),
                       "dsa3d_bwd");
}

}  // namespace

extern "C" {

int msd_abi_version(void) { return MSD_ABI_VERSION; }

const char* msd_last_error(void) { return g_err; }

int msd_dsa3d_fwd(const msd_dsa3d_desc* desc, const void* q, const void* k, const void* v,
                  const void* offsets, const void* extra_k, const void* extra_v, void* out,
                  float* lse, void* stream) {
  int rc = check_dsa(desc);
  if (rc != MSD_OK) return rc;
  rc = check_ptrs("dsa3d_fwd", elem_bytes(desc->dtype), {q, k, v, offsets, out});
  if (rc != MSD_OK) return rc;
  if (desc->extra_g > 0) {
    rc = check_ptrs("dsa3d_fwd(extra_k, extra_v)", 16, {extra_k, extra_v});
    if (rc != MSD_OK) return rc;
  }
  if (lse != nullptr && !aligned(lse, 4)) return fail(MSD_ERR_ALIGN, "dsa3d_fwd: lse misaligned");
  const bool tiled_ok = msd::dsa3d_tiled_supported(*desc, q, k, v);
  if (desc->algo == MSD_ALGO_TILED && !tiled_ok)
    return fail(MSD_ERR_UNSUPPORTED,
                "dsa3d_fwd: tiled kernels need bf16 or fp32, head_dim 32, 64, 96 or 128, <= 160 taps, "
                "<= 256 extra keys and 16-byte aligned rows");
  if (desc->B == 0) return MSD_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (tiled_ok && desc->algo != MSD_ALGO_DIRECT)
    return launch_status(msd::launch_dsa3d_fwd_tiled(*desc, q, k, v, offsets, extra_k, extra_v,
                                                     out, lse, s),
                         "dsa3d_fwd");
  return launch_status(msd::launch_dsa3d_fwd_direct(*desc, q, k, v, offsets, extra_k, extra_v, out,
                                                    lse, s),
                       "dsa3d_fwd");
}

size_t msd_dsa3d_bwd_workspace_size(const msd_dsa3d_desc* desc) {
  if (check_dsa(desc) != MSD_OK) return 0;
  return msd::dsa3d_bwd_ws_bytes(*desc);
}

int msd_dsa3d_bwd(const msd_dsa3d_desc* desc, const void* q, const void* k, const void* v,
                  const void* offsets, const void* extra_k, const void* extra_v, const void* out,
                  const void* dout, const float* lse, const float* dlse, void* dq, void* dk,
                  void* dv, void* doffsets, void* d_extra_k, void* d_extra_v, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return dsa3d_bwd_impl(desc, q, k, v, offsets, extra_k, extra_v, out, dout, lse, dlse, dq, dk, dv,
                        doffsets, d_extra_k, d_extra_v, workspace, workspace_bytes, stream, false);
}

int msd_dsa3d_bwd_noalloc(const msd_dsa3d_desc* desc, const void* q, const void* k,
                          const void* v, const void* offsets, const void* extra_k,
                          const void* extra_v, const void* out, const void* dout,
                          const float* lse, const float* dlse, void* dq, void* dk, void* dv,
                          void* doffsets, void* d_extra_k, void* d_extra_v, void* stream) {
  return dsa3d_bwd_impl(desc, q, k, v, offsets, extra_k, extra_v, out, dout, lse, dlse, dq, dk, dv,
                        doffsets, d_extra_k, d_extra_v, nullptr, 0, stream, true);
}

int msd_dwconv3d_fwd(const msd_dwconv3d_desc* desc, const void* x, const void* weight,
                     const void* bias, void* y, void* preact, void* stream) {
  int rc = check_conv(desc);
  if (rc != MSD_OK) return rc;
  const size_t a = elem_bytes(desc->dtype);
  rc = check_ptrs("dwconv3d_fwd", a, {x, weight, y});
  if (rc != MSD_OK) return rc;
  for (const void* p : {static_cast<const void*>(bias), static_cast<const void*>(preact)})
    if (p != nullptr && !aligned(p, a)) return fail(MSD_ERR_ALIGN, "dwconv3d_fwd: misaligned");
  if (preact != nullptr && desc->act != 1)
    return fail(MSD_ERR_ARG, "dwconv3d_fwd: preact is the GELU input (act = 1 only)");
  if (desc->B == 0) return MSD_OK;
  return launch_status(msd::launch_dwconv3d_fwd(*desc, x, weight, bias, y, preact,
                                                static_cast<hipStream_t>(stream)),
                       "dwconv3d_fwd");
}

size_t msd_dwconv3d_bwd_workspace_size(const msd_dwconv3d_desc* desc) {
  if (check_conv(desc) != MSD_OK) return 0;
  return msd::dwconv3d_bwd_ws_bytes(*desc);
}

int msd_dwconv3d_bwd(const msd_dwconv3d_desc* desc, const void* x, const void* weight,
                     const void* bias, const void* preact, const void* dy, void* dx,
                     void* dweight, void* dbias, void* workspace, size_t workspace_bytes,
                     void* stream) {
  int rc = check_conv(desc);
  if (rc != MSD_OK) return rc;
  const size_t a = elem_bytes(desc->dtype);
  rc = check_ptrs("dwconv3d_bwd", a, {x, weight, dy});
  if (rc != MSD_OK) return rc;
  for (const void* p : {static_cast<const void*>(bias), static_cast<const void*>(dx),
                        static_cast<const void*>(dweight), static_cast<const void*>(dbias),
                        preact})
    if (p != nullptr && !aligned(p, a)) return fail(MSD_ERR_ALIGN, "dwconv3d_bwd: misaligned");
  if (preact != nullptr && desc->act != 1)
    return fail(MSD_ERR_ARG, "dwconv3d_bwd: preact is the GELU input (act = 1 only)");
  if (desc->B == 0) return MSD_OK;
  const size_t need = msd::dwconv3d_bwd_ws_bytes(*desc);
  if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 16))
    return fail(MSD_ERR_WORKSPACE,
                "dwconv3d_bwd: workspace of %zu bytes (16-aligned) needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  return launch_status(msd::launch_dwconv3d_bwd(*desc, x, weight, bias, preact, dy, dx, dweight,
                                                dbias, workspace, static_cast<hipStream_t>(stream)),
                       "dwconv3d_bwd");
}

}  // extern "C"
