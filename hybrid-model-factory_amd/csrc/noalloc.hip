// hmx_gdn_chunk_fwd_noalloc (the GDN prefill without a caller workspace), in a
// code object of its own.
#include <mutex>

#include "common.hpp"

using namespace hmx;

// The no-allocation entry point: hmx_gdn_chunk_fwd with its workspace in a
// file-scope device array instead of a caller buffer.  The array lives in this
// file's code object, which holds no kernel: the runtime loads it (and places the
// array in device memory) the first time a process asks for the array's address,
// i.e. at the first call of this entry point on a device, so processes that never
// call it reserve nothing.  Each device the entry runs on then holds its own copy
// of the array (HMX_GDN_CHUNK_SCRATCH_BYTES) until the process ends.  Nothing in the
// workspace has to start at zero: the planner writes every plan entry, and each
// segment state is written by the S0 / PHI / combine / OUT launches before a
// later launch reads it.  Calls that overlap on one device (concurrent streams or
// threads) share the array and race.
static __device__ __align__(256) unsigned char scratch[HMX_GDN_CHUNK_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];   // the array's device address, per device

// The scratch array's address on the current device, looked up once per device
// (with that device current).  The array's host-side name is not a device
// address: kernels and copies only ever get this pointer.
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(HMX_EHIP, "hmx_gdn_chunk_fwd_noalloc: hipGetDevice failed: %s",
                     hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(HMX_EUNSUPPORTED, "hmx_gdn_chunk_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(HMX_EHIP, "hmx_gdn_chunk_fwd_noalloc: hipGetSymbolAddress(scratch) "
                       "failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_dev[dev] = ptr;
  }
  *out = g_scratch_dev[dev];
  return HMX_OK;
}
}  // namespace

extern "C" int hmx_gdn_chunk_fwd_noalloc(
    const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride, const void* v,
    int64_t v_token_stride, int32_t qkv_dtype, const void* g, int32_t g_dtype, const void* beta,
    int32_t beta_dtype, void* o, const void* h0, void* ht, int64_t state_slot_stride,
    int32_t state_dtype, const int32_t* state_indices, const uint8_t* has_initial_state,
    const int32_t* seg_table, int32_t nseg_total, int32_t N, int32_t H, int32_t HKV, int32_t K,
    int32_t V, float scale, int32_t use_qk_l2norm, int32_t max_warm_chunks,
    float decay_threshold, const hmx_gated_norm* o_norm, const hmx_gate_proj* gates,
    void* stream) {
  HMX_REQUIRE(nseg_total >= 0 && N >= 0 && H > 0, HMX_EINVAL,
              "hmx_gdn_chunk_fwd_noalloc: bad sizes (nseg_total=%d N=%d H=%d)", nseg_total, N, H);
  if (nseg_total == 0) return HMX_OK;
  const size_t need = hmx_gdn_chunk_workspace_bytes(nseg_total, N, H, state_indices != nullptr);
  HMX_REQUIRE(need <= (size_t)HMX_GDN_CHUNK_SCRATCH_BYTES, HMX_EINVAL,
              "hmx_gdn_chunk_fwd_noalloc: this segment table needs %zu bytes of workspace; the "
              "static scratch holds %zu (use fewer segments, or hmx_gdn_chunk_fwd with a "
              "workspace)", need, (size_t)HMX_GDN_CHUNK_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != HMX_OK) return rc;
  return hmx_gdn_chunk_fwd(q, q_token_stride, k, k_token_stride, v, v_token_stride, qkv_dtype, g,
                           g_dtype, beta, beta_dtype, o, h0, ht, state_slot_stride, state_dtype,
                           state_indices, has_initial_state, seg_table, nseg_total, N, H, HKV, K,
                           V, scale, use_qk_l2norm, max_warm_chunks, decay_threshold, ws,
                           (size_t)HMX_GDN_CHUNK_SCRATCH_BYTES, o_norm, gates, stream);
}
