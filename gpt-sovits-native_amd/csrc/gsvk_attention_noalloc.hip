// gsvk_attention_noalloc.hip — decode attention for callers that cannot allocate (code under HIP
// graph capture, serving loops that forbid hipMalloc): gsvk_decode_attention with its key-chunk
// states in a library-owned device array instead of a caller workspace. Same kernels, same
// partition of the keys, so the same bits as gsvk_decode_attention with a large enough workspace.
#include <mutex>

#include "gsvk_common.hpp"

namespace gsvk {

__attribute__((visibility("hidden"))) int attention_call(
                   int kv_dtype, int out_dtype, const float* qkv, size_t ldq, void* k_cache,
                   void* v_cache, size_t max_len, const int64_t* pos, void* out, size_t ldo,
                   size_t batch, size_t heads, size_t head_dim, size_t len_bound, void* workspace,
                   size_t workspace_bytes, bool need_ws, int32_t* err, void* stream);

namespace {

// The chunk states, one copy per GPU, held until the process ends: B x C x 3 KiB for C > 1 key
// chunks (one chunk needs none). 4 MiB holds 1365 states: on a 256-CU device every batch of up to
// 256 sequences at any length (B x C <= 256 there) and up to 682 sequences at contexts of at most
// 256 keys (C <= 2); a call that needs more is rejected (GSVK_E_SIZE). Every call on a GPU shares
// its copy. The chunk kernel
// writes every state the merge kernel reads, so nothing needs clearing between calls; two calls in
// flight at once on one GPU (different streams) race on it.
constexpr size_t kScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of this GPU's `scratch`, looked up once per device with that device current. In
// host code the array's name is only a stand-in for the symbol: kernels and copies get this
// address. Null when the lookup fails.
void* scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace
}  // namespace gsvk

using namespace gsvk;

extern "C" int gsvk_decode_attention_noalloc(int kv_dtype, int out_dtype, const float* qkv,
                                             size_t ldq, void* k_cache, void* v_cache,
                                             size_t max_len, const int64_t* pos, void* out,
                                             size_t ldo, size_t batch, size_t heads,
                                             size_t head_dim, size_t len_bound, int32_t* err,
                                             void* stream) {
  void* ws = scratch_ptr();
  if (!ws) return GSVK_E_HIP;
  return attention_call(kv_dtype, out_dtype, qkv, ldq, k_cache, v_cache, max_len, pos, out, ldo,
                        batch, heads, head_dim, len_bound, ws, kScratchBytes, true, err, stream);
}
