// Sparse-attention backward that allocates nothing: si_sparse_attn_bwd_ragged
// run on a workspace that is a file-scope device array instead of a
// caller-provided buffer.  For callers that cannot allocate device memory
// (code under HIP graph capture, tight training loops, harnesses that forbid
// hipMalloc).
//
// Each GPU the library runs on holds its own copy of `scratch` from module
// load until the process ends.  On the host, the array's name is a stand-in,
// not a device address: the device address comes from hipGetSymbolAddress,
// looked up once per device (on the first call made on that device, with that
// device current) and kept in g_scratch_ptr.  Every call on one GPU shares
// that GPU's array and leaves its contents behind; the backward writes every
// workspace region before reading it (segment bounds are filled, the first
// row chunk writes the key accumulator, every row writes its dsink terms), so
// nothing has to start at zero.  Calls that overlap on one GPU (other host
// threads, other streams) race on the array.
#include <mutex>
#include <string>

#include "si_status.h"

namespace si {

static constexpr int64_t kNoAllocScratchBytes = int64_t{128} << 20;
static constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kNoAllocMaxDevices] = {};

// Device address of the current device's `scratch`.
static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SI_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kNoAllocMaxDevices) return set_error(SI_ERR_UNSUPPORTED, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SI_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SI_OK;
}

}  // namespace si

using namespace si;

extern "C" int64_t si_sparse_attn_bwd_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int si_sparse_attn_bwd_noalloc(const void* q, const int64_t* q_strides, const void* kv,
                                          const int64_t* kv_strides, const float* attn_sink, const void* topk_idxs,
                                          int idx_is_i64, const int64_t* idx_strides, const void* o,
                                          const int64_t* o_strides, const float* lse, const int64_t* lse_strides,
                                          const void* dout, const int64_t* do_strides, int64_t B, int64_t S,
                                          int64_t H, int64_t D, int64_t N_kv, int64_t K, float softmax_scale,
                                          int qkv_dtype, void* dq, const int64_t* dq_strides, void* dkv,
                                          const int64_t* dkv_strides, float* dsink, const int32_t* row_len,
                                          const int64_t* row_len_strides, void* stream) {
  // What the plan for this problem needs within the scratch: its whole
  // workspace if that fits, else the smallest (one query row per chunk).
  if (B < 0 || S < 0 || H <= 0 || D <= 0 || N_kv < 0 || K < 0) return set_error(SI_ERR_INVALID, "bad dimension");
  const int64_t need = si_sparse_attn_bwd_workspace_bytes(B, S, H, D, N_kv, K, kNoAllocScratchBytes);
  if (need < 0) return SI_ERR_UNSUPPORTED;  // si_last_error() holds the reason (head dim, int32 range)
  if (need > kNoAllocScratchBytes)
    return set_error(SI_ERR_UNSUPPORTED,
                     "problem too large for the no-alloc backward: one query row needs " + std::to_string(need) +
                         " bytes of workspace, the static scratch holds " + std::to_string(kNoAllocScratchBytes) +
                         " (use si_sparse_attn_bwd_ragged with a caller-provided workspace)");
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return si_sparse_attn_bwd_ragged(q, q_strides, kv, kv_strides, attn_sink, topk_idxs, idx_is_i64, idx_strides, o,
                                   o_strides, lse, lse_strides, dout, do_strides, B, S, H, D, N_kv, K, softmax_scale,
                                   qkv_dtype, dq, dq_strides, dkv, dkv_strides, dsink, ws, kNoAllocScratchBytes, row_len,
                                   row_len_strides, stream);
}
