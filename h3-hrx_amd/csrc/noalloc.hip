// h3_attention_i8qk_static: h3_attention_i8qk_ws for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc) and have
// none to lend. The workspace (the head-major copy of the key scales) is a file-scope device
// array of kScratchBytes instead of a caller's buffer; everything else is the _ws form's code.
//
// `scratch` below is a device symbol: in host code its name is a stand-in, not a device address,
// so the host never passes it to a kernel or a copy. Once per device, on the first call with that
// device current, hipGetSymbolAddress gives that device's copy of the array (each GPU holds its
// own, at its own address, until the process ends); the address is kept per device and is what
// the kernels receive. After that set-up a call allocates nothing and calls no allocating
// routine. Calls on one device share its array, which keeps the last call's contents (the
// transpose writes every scale a call's attention kernel reads, so nothing has to start at zero);
// calls that overlap on one device (different streams, no ordering between them) race on it.
#include <mutex>

#include "internal.hpp"

namespace h3 {
namespace {

constexpr size_t kScratchBytes = size_t{8} << 20;  // 8 MiB: up to 2,097,152 key scales
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // per device: the address of its `scratch`, once known

// The current device's copy of `scratch` (its address looked up on first use).
int device_scratch(const char* stage, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(H3_ERR_NO_DEVICE, "%s: no current HIP device (%s)", stage,
                     hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(H3_ERR_NO_DEVICE, "%s: device %d beyond the %d this library tracks", stage,
                     dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(H3_ERR_LAUNCH, "%s: hipGetSymbolAddress of the scratch array failed (%s)",
                       stage, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return H3_OK;
}

}  // namespace
}  // namespace h3

extern "C" int h3_attention_i8qk_static(const h3_attention_cfg* cfg, uint32_t token_count,
                                        uint32_t heads, h3_view qi, h3_view qs, h3_view ki,
                                        h3_view ks, h3_view vt, h3_view out, h3_stream stream) {
  using namespace h3;
  const char* stage = "attention_i8qk_static";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  const size_t need = scales_workspace_bytes(*cfg);
  if (need > kScratchBytes)
    return set_error(H3_ERR_CONFIG,
                     "%s: (kv_stride/128) * tokens * 4 = %zu bytes of key scales exceed the %zu-byte "
                     "static scratch (use h3_attention_i8qk_ws with a lent workspace)",
                     stage, need, kScratchBytes);
  void* ptr = nullptr;
  int st = device_scratch(stage, &ptr);
  if (st) return st;
  return attention_i8qk_static_ws(cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                                  h3_view{ptr, kScratchBytes}, reinterpret_cast<hipStream_t>(stream));
}
