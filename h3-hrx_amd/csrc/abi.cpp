// C ABI of libh3attn (include/h3attn.h): argument and binding checks, then the HIP launchers.
//
// Every entry point validates before it touches the device, exactly as the reference's
// dispatch::emit checks bindings before dispatch (src/dispatch.rs:264-276) and as each Loom
// kernel's config.decl ranges bound its specialisation (kernels/*.loom). A failing check
// returns its status, records a message for h3_last_error(), and launches nothing.
#include <algorithm>
#include <cstdarg>
#include <initializer_list>
#include <cstdio>
#include <string>

#include "internal.hpp"

namespace h3 {

static std::string& g_error_ref() {
  thread_local std::string e;
  return e;
}

int set_error(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error_ref() = buf;
  return status;
}

namespace {

int ok() {
  g_error_ref().clear();
  return H3_OK;
}

// src/dispatch.rs:264-276: every binding must cover the extent the kernel addresses.
int check_bindings(const char* stage, const h3_view* views, const size_t* need, int n) {
  for (int i = 0; i < n; ++i) {
    if (views[i].bytes < need[i])
      return set_error(H3_ERR_BINDING, "%s: binding %d is %zu bytes, the kernel addresses %zu", stage, i,
                  views[i].bytes, need[i]);
    if (need[i] > 0 && views[i].ptr == nullptr)
      return set_error(H3_ERR_ARGUMENT, "%s: binding %d is null", stage, i);
  }
  // With a device present, every binding must be memory the current device can address: a host
  // pointer or another device's buffer handed to a kernel faults the GPU. The HIP runtime knows
  // this process's allocations (device, managed and pinned host memory); anything else it
  // refuses. On a host with no device, device_ready() reports that instead.
  int devices = 0, current = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
    (void)hipGetLastError();
    return H3_OK;
  }
  if (hipGetDevice(&current) != hipSuccess) {
    (void)hipGetLastError();
    return H3_OK;
  }
  for (int i = 0; i < n; ++i) {
    if (need[i] == 0) continue;
    hipPointerAttribute_t attr{};
    const hipError_t e = hipPointerGetAttributes(&attr, views[i].ptr);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(H3_ERR_ARGUMENT, "%s: binding %d is not memory the device can address (%s)",
                       stage, i, hipGetErrorString(e));
    }
    if (attr.type == hipMemoryTypeDevice && attr.device != current)
      return set_error(H3_ERR_ARGUMENT, "%s: binding %d lives on device %d, the current device is %d",
                       stage, i, attr.device, current);
  }
  return H3_OK;
}

// The row kernels (quantizers, VSA rows) move 16 bytes (eight 16-bit channels) per access.
int check_aligned16(const char* stage, std::initializer_list<h3_view> views) {
  int i = 0;
  for (const h3_view& v : views) {
    if (reinterpret_cast<uintptr_t>(v.ptr) % 16 != 0)
      return set_error(H3_ERR_ARGUMENT, "%s: binding %d is not 16-byte aligned", stage, i);
    ++i;
  }
  return H3_OK;
}

// config.decl ... where [range(v, lo, hi), multiple_of(v, m)]: lo <= v <= hi, v % m == 0.
bool in_range(uint32_t v, uint32_t lo, uint32_t hi, uint32_t multiple = 1) {
  return v >= lo && v <= hi && v % multiple == 0;
}

int launched(const char* stage, hipError_t e) {
  if (e != hipSuccess) return set_error(H3_ERR_LAUNCH, "%s: %s", stage, hipGetErrorString(e));
  return ok();
}

int device_ready(const char* stage) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return set_error(H3_ERR_NO_DEVICE, "%s: no HIP device (%s)", stage, hipGetErrorString(e));
  return H3_OK;
}

// kernels/prepare_qk_i8.loom:9-15 (+ prepare_qk_i8hm.loom:13, prepare_qk_rope_i8hm.loom:15-17)
int check_prepare_cfg(const char* stage, const h3_prepare_cfg* cfg, uint32_t tokens,
                      bool head_major) {
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  if (!in_range(cfg->row_stride, 128, 65536, 128))
    return set_error(H3_ERR_CONFIG, "%s: row_stride %u outside [128, 65536] step 128", stage,
                cfg->row_stride);
  if (!in_range(cfg->head_offset, 0, 65536, 128))
    return set_error(H3_ERR_CONFIG, "%s: head_offset %u outside [0, 65536] step 128", stage,
                cfg->head_offset);
  if (!in_range(cfg->heads, 1, 256))
    return set_error(H3_ERR_CONFIG, "%s: heads %u outside [1, 256]", stage, cfg->heads);
  if ((uint64_t)cfg->head_offset + 128ull * cfg->heads > cfg->row_stride)
    return set_error(H3_ERR_CONFIG, "%s: head_offset %u + %u heads exceed row_stride %u", stage,
                cfg->head_offset, cfg->heads, cfg->row_stride);
  if (cfg->elem != H3_ELEM_F16 && cfg->elem != H3_ELEM_BF16)
    return set_error(H3_ERR_CONFIG, "%s: unknown element format %u", stage, cfg->elem);
  if (!in_range(tokens, 1, 1048576))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 1048576]", stage, tokens);
  if (head_major) {
    if (!in_range(cfg->token_capacity, 32, 1048576, 32))
      return set_error(H3_ERR_CONFIG, "%s: token_capacity %u outside [32, 1048576] step 32", stage,
                  cfg->token_capacity);
    // "The host's capacity is at least tokens + 16, so a token's scale row is in bounds."
    // (prepare_qk_i8hm.loom in-file 51-53): the kernel addresses rows < token_capacity.
    if (tokens > cfg->token_capacity)
      return set_error(H3_ERR_ARGUMENT, "%s: tokens %u exceed token_capacity %u", stage, tokens,
                  cfg->token_capacity);
  }
  return H3_OK;
}

int prepare_common(const char* stage, const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x,
                   h3_view mean, h3_view codes, h3_view scales, hipStream_t stream,
                   bool head_major) {
  int st = check_prepare_cfg(stage, cfg, tokens, head_major);
  if (st) return st;
  const size_t rows_out = head_major ? (size_t)cfg->heads * cfg->token_capacity
                                     : (size_t)tokens * cfg->heads;
  h3_view views[4] = {x, mean, codes, scales};
  size_t need[4] = {(size_t)tokens * cfg->row_stride * 2, mean.ptr ? (size_t)cfg->row_stride * 4 : 0,
                    rows_out * 128, rows_out * 4};
  if ((st = check_bindings(stage, views, need, 4))) return st;
  if ((st = check_aligned16(stage, {x, mean}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_prepare_qk(*cfg, tokens, head_major, x.ptr,
                                           static_cast<const float*>(mean.ptr),
                                           static_cast<int32_t*>(codes.ptr),
                                           static_cast<float*>(scales.ptr), stream));
}

int rope_bindings(const char* stage, const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x,
                  h3_view weight, h3_view cos_t, h3_view sin_t) {
  h3_view views[4] = {x, weight, cos_t, sin_t};
  size_t need[4] = {(size_t)tokens * cfg->row_stride * 2, 128 * 4, (size_t)tokens * 48 * 4,
                    (size_t)tokens * 48 * 4};
  const int st = check_bindings(stage, views, need, 4);
  return st ? st : check_aligned16(stage, {x, weight, cos_t, sin_t});
}

// Operand layouts of the attention kernels (attention.hip's modes).
enum {
  kModeTokenI8 = 0,
  kModeHeadI8 = 1,
  kModeTokenI4 = 2,
  kModeTokenI4Skip = 3,
  kModeTokenI8Vsa = 4,
  kModeTokenI4Fp6 = 5
};

// The attention config (kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:7-17 and the same
// declarations in vsa_attention_16.loom) and the launch arguments every attention form shares.
int check_attention_cfg(const char* stage, const h3_attention_cfg* cfg, uint32_t token_count,
                        uint32_t heads) {
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  // kernels/attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:7-17
  if (!in_range(cfg->q_stride, 128, 32768, 128))
    return set_error(H3_ERR_CONFIG, "%s: q_stride %u outside [128, 32768] step 128", stage,
                cfg->q_stride);
  if (!in_range(cfg->kv_stride, 128, 32768, 128))
    return set_error(H3_ERR_CONFIG, "%s: kv_stride %u outside [128, 32768] step 128", stage,
                cfg->kv_stride);
  if (!in_range(cfg->out_stride, 128, 32768, 128))
    return set_error(H3_ERR_CONFIG, "%s: out_stride %u outside [128, 32768] step 128", stage,
                cfg->out_stride);
  if (!in_range(cfg->tokens, 1, 1048576))
    return set_error(H3_ERR_CONFIG, "%s: tokens %u outside [1, 1048576]", stage, cfg->tokens);
  if (!in_range(cfg->token_capacity, 32, 1048576, 16))
    return set_error(H3_ERR_CONFIG, "%s: token_capacity %u outside [32, 1048576] step 16", stage,
                cfg->token_capacity);
  if (cfg->tokens > cfg->token_capacity)
    return set_error(H3_ERR_CONFIG, "%s: tokens %u exceed token_capacity %u", stage, cfg->tokens,
                cfg->token_capacity);
  if (token_count < 1 || token_count > cfg->tokens)
    return set_error(H3_ERR_ARGUMENT, "%s: token_count %u outside [1, tokens=%u]", stage, token_count,
                cfg->tokens);
  if (heads < 1 || heads > 65535)
    return set_error(H3_ERR_ARGUMENT, "%s: heads %u outside [1, 65535]", stage, heads);
  return H3_OK;
}

// The heads a launch touches. Workgroup row y of the [.., heads] workload takes key/value head
// y % (kv_stride/128) and query head kv_head % (out_stride/128)
// (attention_i8qkhm_mha8_k64_lds_f16_wmma.loom:300-340, attention_i8qk_family.loom:77-91), so
// the key/value heads 0..kv-1 and the query heads 0..q-1 are read, with kv = min(heads,
// kv_stride/128) and q = min(kv, out_stride/128). A padded output pitch (out_stride above
// heads*128, src/stack.rs:751-758) therefore reads no more query heads than the launch has; the
// binding extents below follow these counts, as the reference's caller sizes its operands by
// the workload's heads (src/stack.rs:1830-1837).
struct TouchedHeads {
  size_t q, kv;
};
TouchedHeads touched_heads(const h3_attention_cfg& cfg, uint32_t heads) {
  const size_t kv = std::min<size_t>(heads, cfg.kv_stride / 128);
  return {std::min<size_t>(kv, cfg.out_stride / 128), kv};
}

int attention_common(const char* stage, const h3_attention_cfg* cfg, uint32_t token_count,
                     uint32_t heads, h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                     h3_view out, hipStream_t stream, int mode, float skip_tau = 0.0f,
                     h3_view routes = {}, h3_view lengths = {}, h3_view workspace = {},
                     bool static_workspace = false) {
  const bool head_major = mode == kModeHeadI8;
  const bool vsa = mode == kModeTokenI8Vsa;
  const bool fp6 = mode == kModeTokenI4Fp6;
  const size_t code_div = (mode == kModeTokenI4 || mode == kModeTokenI4Skip || fp6) ? 2 : 1;
  int st = check_attention_cfg(stage, cfg, token_count, heads);
  if (st) return st;
  const size_t cap = cfg->token_capacity;
  const TouchedHeads th = touched_heads(*cfg, heads);
  // Token-major code rows hold q_stride/128 query heads; a launch whose query heads lie past a
  // row would read the next token's codes (the reference assumes it away,
  // attention_i8qk_family.loom:160-170).
  if (!head_major && th.q > cfg->q_stride / 128)
    return set_error(H3_ERR_CONFIG, "%s: q_stride %u holds %u query heads, the launch reads %zu",
                     stage, cfg->q_stride, cfg->q_stride / 128, th.q);
  // The extents the kernel addresses. Head-major: codes [head*cap + t][32] i32 and scales
  // [head][cap] f32 of the touched heads (attention_i8qkhm...loom:394-401). Token-major: whole
  // rows [cap][q_stride/4] i32 and [cap][q_stride/128] f32, and the same for K
  // (attention_i8qk_family.loom:108-113). V^T: the 128 rows of every touched key/value head,
  // [kv_stride][cap] f16. Output: rows < token_count at out_stride, the touched heads' columns.
  size_t need[6];
  if (head_major) {
    need[0] = th.q * cap * 128;
    need[1] = th.q * cap * 4;
    need[2] = th.kv * cap * 128;
    need[3] = th.kv * cap * 4;
  } else {
    need[0] = cap * cfg->q_stride / code_div;
    need[1] = cap * (cfg->q_stride / 128) * 4;
    need[2] = cap * cfg->kv_stride / code_div;
    need[3] = cap * (cfg->kv_stride / 128) * 4;
  }
  need[4] = th.kv * 128 * cap * 2;
  need[5] = ((size_t)(token_count - 1) * cfg->out_stride + th.q * 128) * 2;
  h3_view views[6] = {qi, qs, ki, ks, vt, out};
  st = check_bindings(stage, views, need, 6);
  if (st) return st;
  // A workspace (token-major operands) receives a head-major copy of the key scales (or the FP6
  // operands), which the kernel then reads; without one it reads them token-major. Nothing is
  // allocated either way. A lent workspace is device memory like any binding and goes through
  // the same checks; the library's own static array (h3_attention_i8qk_static) is known good.
  if (workspace.ptr) {
    const size_t ws_need = fp6 ? fp6_layout(*cfg).bytes : scales_workspace_bytes(*cfg);
    if (static_workspace) {
      if (workspace.bytes < ws_need)
        return set_error(H3_ERR_BINDING, "%s: workspace is %zu bytes, the kernel addresses %zu",
                         stage, workspace.bytes, ws_need);
    } else {
      h3_view wv[1] = {workspace};
      size_t wneed[1] = {ws_need};
      if ((st = check_bindings(stage, wv, wneed, 1)))
        return st == H3_ERR_BINDING
                   ? set_error(H3_ERR_BINDING, "%s: workspace is %zu bytes, the kernel addresses %zu",
                               stage, workspace.bytes, ws_need)
                   : st;
    }
  }
  if (vsa) {
    // kernels/vsa_attention_8.loom:145-150: blocks = tokens / 64, routes [heads][blocks][blocks]
    // i32, lengths [blocks] i32. Whole cubes only: tokens is the padded row count.
    if (cfg->tokens % 64 != 0 || cfg->tokens / 64 > 16384)
      return set_error(H3_ERR_CONFIG, "%s: tokens %u is not 64 * blocks with blocks <= 16384",
                       stage, cfg->tokens);
    const size_t blocks = cfg->tokens / 64;
    h3_view rv[2] = {routes, lengths};
    size_t rneed[2] = {th.q * blocks * blocks * 4, blocks * 4};
    if ((st = check_bindings(stage, rv, rneed, 2))) return st;
    if ((st = device_ready(stage))) return st;
    return launched(stage, launch_attention_vsa(*cfg, token_count, heads,
                                                static_cast<const int32_t*>(qi.ptr),
                                                static_cast<const float*>(qs.ptr),
                                                static_cast<const int32_t*>(ki.ptr),
                                                static_cast<const float*>(ks.ptr),
                                                static_cast<const uint16_t*>(vt.ptr),
                                                static_cast<uint16_t*>(out.ptr),
                                                static_cast<const int32_t*>(routes.ptr),
                                                static_cast<const int32_t*>(lengths.ptr),
                                                workspace.ptr, stream));
  }
  if ((st = device_ready(stage))) return st;
  if (fp6)
    return launched(stage, launch_attention_i4_fp6(*cfg, token_count, heads,
                                                   static_cast<const int32_t*>(qi.ptr),
                                                   static_cast<const float*>(qs.ptr),
                                                   static_cast<const int32_t*>(ki.ptr),
                                                   static_cast<const float*>(ks.ptr),
                                                   static_cast<const uint16_t*>(vt.ptr),
                                                   static_cast<uint16_t*>(out.ptr), workspace.ptr,
                                                   stream));
  return launched(stage, launch_attention(*cfg, mode, skip_tau, token_count, heads,
                                          static_cast<const int32_t*>(qi.ptr),
                                          static_cast<const float*>(qs.ptr),
                                          static_cast<const int32_t*>(ki.ptr),
                                          static_cast<const float*>(ks.ptr),
                                          static_cast<const uint16_t*>(vt.ptr),
                                          static_cast<uint16_t*>(out.ptr), workspace.ptr,
                                          stream));
}

// kernels/vsa_ops.loom:3-9 (h3.vsa.*), plus the relations src/vsa/device.rs:63-77 builds the
// config with: padded = 64 * blocks, width = 128 * heads, prefix <= blocks.
int check_vsa_cfg(const char* stage, const h3_vsa_cfg* cfg) {
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  if (!in_range(cfg->tokens, 1, 1048576))
    return set_error(H3_ERR_CONFIG, "%s: tokens %u outside [1, 1048576]", stage, cfg->tokens);
  if (!in_range(cfg->padded, 64, 1048576, 64))
    return set_error(H3_ERR_CONFIG, "%s: padded %u outside [64, 1048576] step 64", stage,
                     cfg->padded);
  if (!in_range(cfg->width, 128, 32768, 128))
    return set_error(H3_ERR_CONFIG, "%s: width %u outside [128, 32768] step 128", stage,
                     cfg->width);
  if (!in_range(cfg->blocks, 1, 16384) || cfg->padded != 64 * cfg->blocks)
    return set_error(H3_ERR_CONFIG, "%s: blocks %u outside [1, 16384] or not padded/64 (%u)",
                     stage, cfg->blocks, cfg->padded / 64);
  if (!in_range(cfg->heads, 1, 256) || cfg->width != 128 * cfg->heads)
    return set_error(H3_ERR_CONFIG, "%s: heads %u outside [1, 256] or not width/128", stage,
                     cfg->heads);
  if (cfg->prefix > cfg->blocks)
    return set_error(H3_ERR_CONFIG, "%s: prefix %u exceeds blocks %u", stage, cfg->prefix,
                     cfg->blocks);
  if (cfg->topk > 16384)
    return set_error(H3_ERR_CONFIG, "%s: topk %u outside [0, 16384]", stage, cfg->topk);
  return H3_OK;
}


int transpose_common(const char* stage, const h3_transpose_cfg* cfg, uint32_t launch_rows,
                     uint32_t rows, h3_view x, h3_view out, hipStream_t stream, bool qkv) {
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  // kernels/transpose_f16.loom:7-9
  if (!in_range(cfg->width, 32, 65536, 32))
    return set_error(H3_ERR_CONFIG, "%s: width %u outside [32, 65536] step 32", stage, cfg->width);
  if (!in_range(cfg->row_capacity, 32, 1048576, 32))
    return set_error(H3_ERR_CONFIG, "%s: row_capacity %u outside [32, 1048576] step 32", stage,
                cfg->row_capacity);
  if (cfg->elem != H3_ELEM_F16 && cfg->elem != H3_ELEM_BF16)
    return set_error(H3_ERR_CONFIG, "%s: unknown element format %u", stage, cfg->elem);
  // range(%rows, 1, 1048576), le(%rows, %cap) (transpose_f16.loom in-file 34)
  if (rows < 1 || rows > cfg->row_capacity || launch_rows < rows ||
      launch_rows > cfg->row_capacity)
    return set_error(H3_ERR_ARGUMENT, "%s: rows %u / launch_rows %u outside [1, row_capacity=%u]",
                stage, rows, launch_rows, cfg->row_capacity);
  const uint32_t stride = qkv ? 3 * cfg->width : cfg->width;
  h3_view views[2] = {x, out};
  size_t need[2] = {(size_t)rows * stride * 2, (size_t)cfg->width * cfg->row_capacity * 2};
  int st = check_bindings(stage, views, need, 2);
  if (st) return st;
  if ((st = device_ready(stage))) return st;
  const uint32_t tile = (qkv && cfg->width % 64 == 0) ? 64 : 32;
  return launched(stage, launch_transpose(cfg->width, cfg->row_capacity, stride,
                                          qkv ? 2 * cfg->width : 0, cfg->elem, tile, launch_rows,
                                          rows, x.ptr, static_cast<uint16_t*>(out.ptr), stream));
}

}  // namespace

int attention_i8qk_static_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                             h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                             h3_view out, h3_view workspace, hipStream_t stream) {
  return attention_common("attention_i8qk_static", cfg, token_count, heads, qi, qs, ki, ks, vt,
                          out, stream, kModeTokenI8, 0.0f, {}, {}, workspace, true);
}

int vsa_attention_i8_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_view routes, h3_view lengths, h3_view workspace, hipStream_t stream) {
  return attention_common("VSA attention", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          stream, kModeTokenI8Vsa, 0.0f, routes, lengths, workspace);
}

int vsa_gather_pool(const h3_vsa_cfg* cfg, h3_view src, h3_view lengths, h3_view x, h3_view y,
                    h3_view means, h3_stream stream) {
  const char* stage = "VSA gather";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, t = cfg->tokens, w = cfg->width, b = cfg->blocks;
  h3_view views[5] = {src, x, y, lengths, means};
  size_t need[5] = {n * 4, t * w * 2, n * w * 2, b * 4, b * w * 4};
  if ((st = check_bindings(stage, views, need, 5))) return st;
  if ((st = check_aligned16(stage, {x, y, means}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_gather_pool(cfg->tokens, cfg->blocks, cfg->width,
                                                static_cast<const int32_t*>(src.ptr),
                                                static_cast<const int32_t*>(lengths.ptr),
                                                static_cast<const uint16_t*>(x.ptr),
                                                static_cast<uint16_t*>(y.ptr),
                                                static_cast<float*>(means.ptr),
                                                reinterpret_cast<hipStream_t>(stream)));
}

int vsa_gather_transpose(const h3_vsa_cfg* cfg, h3_view src, h3_view x, h3_view y, h3_view vt,
                         h3_stream stream) {
  const char* stage = "VSA gather";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, t = cfg->tokens, w = cfg->width;
  h3_view views[4] = {src, x, y, vt};
  size_t need[4] = {n * 4, t * w * 2, n * w * 2, w * n * 2};
  if ((st = check_bindings(stage, views, need, 4))) return st;
  if ((st = check_aligned16(stage, {x, y}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_gather_transpose(cfg->width, cfg->padded,
                                                 static_cast<const int32_t*>(src.ptr),
                                                 cfg->tokens,
                                                 static_cast<const uint16_t*>(x.ptr),
                                                 static_cast<uint16_t*>(y.ptr),
                                                 static_cast<uint16_t*>(vt.ptr),
                                                 reinterpret_cast<hipStream_t>(stream)));
}
}  // namespace h3

using namespace h3;

extern "C" {

const char* h3_last_error(void) { return g_error_ref().c_str(); }

const char* h3_version(void) { return "h3attn 0.1.0 gfx950"; }

int h3_prepare_qk_i8(const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x, h3_view mean,
                     h3_view codes, h3_view scales, h3_stream stream) {
  return prepare_common("prepare_qk_i8", cfg, tokens, x, mean, codes, scales,
                        reinterpret_cast<hipStream_t>(stream), false);
}

int h3_prepare_qk_i8hm(const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x, h3_view mean,
                       h3_view codes, h3_view scales, h3_stream stream) {
  return prepare_common("prepare_qk_i8hm", cfg, tokens, x, mean, codes, scales,
                        reinterpret_cast<hipStream_t>(stream), true);
}

int h3_prepare_qk_i4(const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x, h3_view mean,
                     h3_view codes, h3_view scales, h3_stream stream) {
  const char* stage = "prepare_qk_i4";
  // kernels/prepare_qk_i4.loom:11-17 (token-major; token_capacity is not read)
  int st = check_prepare_cfg(stage, cfg, tokens, false);
  if (st) return st;
  const size_t rows_out = (size_t)tokens * cfg->heads;
  h3_view views[4] = {x, mean, codes, scales};
  size_t need[4] = {(size_t)tokens * cfg->row_stride * 2, mean.ptr ? (size_t)cfg->row_stride * 4 : 0,
                    rows_out * 64, rows_out * 4};
  if ((st = check_bindings(stage, views, need, 4))) return st;
  if ((st = check_aligned16(stage, {x, mean}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_prepare_qk_i4(*cfg, tokens, x.ptr,
                                              static_cast<const float*>(mean.ptr),
                                              static_cast<int32_t*>(codes.ptr),
                                              static_cast<float*>(scales.ptr),
                                              reinterpret_cast<hipStream_t>(stream)));
}

int h3_prepare_qk_rope_i8hm(const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x,
                            h3_view weight, h3_view cos_t, h3_view sin_t, h3_view codes,
                            h3_view scales, h3_stream stream) {
  const char* stage = "prepare_qk_rope_i8hm";
  int st = check_prepare_cfg(stage, cfg, tokens, true);
  if (st) return st;
  if ((st = rope_bindings(stage, cfg, tokens, x, weight, cos_t, sin_t))) return st;
  const size_t rows_out = (size_t)cfg->heads * cfg->token_capacity;
  h3_view views[2] = {codes, scales};
  size_t need[2] = {rows_out * 128, rows_out * 4};
  if ((st = check_bindings(stage, views, need, 2))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_prepare_qk_rope(
                             *cfg, tokens, x.ptr, static_cast<const float*>(weight.ptr),
                             static_cast<const float*>(cos_t.ptr),
                             static_cast<const float*>(sin_t.ptr),
                             static_cast<int32_t*>(codes.ptr), static_cast<float*>(scales.ptr),
                             reinterpret_cast<hipStream_t>(stream)));
}

int h3_prepare_k_rope_smooth_i8hm(const h3_prepare_cfg* cfg, uint32_t tokens, h3_view x,
                                  h3_view weight, h3_view cos_t, h3_view sin_t, h3_view mean,
                                  h3_view codes, h3_view scales, h3_stream stream) {
  const char* stage = "prepare_k_rope_smooth_i8hm";
  int st = check_prepare_cfg(stage, cfg, tokens, true);
  if (st) return st;
  if ((st = rope_bindings(stage, cfg, tokens, x, weight, cos_t, sin_t))) return st;
  const size_t rows_out = (size_t)cfg->heads * cfg->token_capacity;
  h3_view views[3] = {mean, codes, scales};
  size_t need[3] = {(size_t)cfg->heads * 128 * 4, rows_out * 128, rows_out * 4};
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = device_ready(stage))) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = launch_rope_colmean(*cfg, tokens, x.ptr, static_cast<const float*>(weight.ptr),
                                     static_cast<const float*>(cos_t.ptr),
                                     static_cast<const float*>(sin_t.ptr),
                                     static_cast<float*>(scales.ptr),
                                     static_cast<float*>(mean.ptr), s);
  if (e != hipSuccess) return launched(stage, e);
  return launched(stage, launch_prepare_qk_rope_mean(
                             *cfg, tokens, x.ptr, static_cast<const float*>(weight.ptr),
                             static_cast<const float*>(cos_t.ptr),
                             static_cast<const float*>(sin_t.ptr),
                             static_cast<const float*>(mean.ptr),
                             static_cast<int32_t*>(codes.ptr), static_cast<float*>(scales.ptr), s));
}

int h3_rope_qknorm_f16(const h3_rope_cfg* cfg, uint32_t tokens, h3_view x, h3_view qweight,
                       h3_view kweight, h3_view cos_t, h3_view sin_t, h3_view q_out,
                       h3_view k_out, h3_view v_out, h3_stream stream) {
  const char* stage = "rope_qknorm_f16";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  if (!in_range(cfg->row_stride, 128, 65536, 128) || !in_range(cfg->heads, 1, 256) ||
      !in_range(cfg->kv_heads, 1, 256) || !in_range(cfg->k_offset, 0, 65536, 128) ||
      cfg->elem > H3_ELEM_BF16)
    return set_error(H3_ERR_CONFIG, "%s: config outside the declared ranges", stage);
  const uint64_t end = (uint64_t)cfg->k_offset + 128ull * cfg->kv_heads * (cfg->copy_v ? 2 : 1);
  if (128ull * cfg->heads > cfg->k_offset || end > cfg->row_stride)
    return set_error(H3_ERR_CONFIG, "%s: heads/kv_heads/k_offset exceed row_stride %u", stage,
                cfg->row_stride);
  if (!in_range(tokens, 1, 1048576))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 1048576]", stage, tokens);
  h3_view views[8] = {x, qweight, kweight, cos_t, sin_t, q_out, k_out, v_out};
  size_t need[8] = {(size_t)tokens * cfg->row_stride * 2,
                    128 * 4,
                    128 * 4,
                    (size_t)tokens * 48 * 4,
                    (size_t)tokens * 48 * 4,
                    (size_t)tokens * cfg->heads * 128 * 2,
                    (size_t)tokens * cfg->kv_heads * 128 * 2,
                    cfg->copy_v ? (size_t)tokens * cfg->kv_heads * 128 * 2 : 0};
  int st = check_bindings(stage, views, need, 8);
  if (st) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_rope_qknorm(
                             *cfg, tokens, x.ptr, static_cast<const float*>(qweight.ptr),
                             static_cast<const float*>(kweight.ptr),
                             static_cast<const float*>(cos_t.ptr),
                             static_cast<const float*>(sin_t.ptr),
                             static_cast<uint16_t*>(q_out.ptr), static_cast<uint16_t*>(k_out.ptr),
                             static_cast<uint16_t*>(v_out.ptr),
                             reinterpret_cast<hipStream_t>(stream)));
}

int h3_colmean_f32(uint32_t width, uint32_t elem, uint32_t tokens, h3_view x, h3_view mean,
                   h3_stream stream) {
  const char* stage = "colmean_f32";
  // kernels/colmean_f32.loom:5
  if (!in_range(width, 256, 65536, 256))
    return set_error(H3_ERR_CONFIG, "%s: width %u outside [256, 65536] step 256", stage, width);
  if (elem > H3_ELEM_BF16) return set_error(H3_ERR_CONFIG, "%s: unknown element format", stage);
  if (!in_range(tokens, 1, 1048576))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 1048576]", stage, tokens);
  h3_view views[2] = {x, mean};
  size_t need[2] = {(size_t)tokens * width * 2, (size_t)width * 4};
  int st = check_bindings(stage, views, need, 2);
  if (st) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_colmean(width, width, elem, tokens, x.ptr,
                                        static_cast<float*>(mean.ptr),
                                        reinterpret_cast<hipStream_t>(stream)));
}

int h3_transpose_f16(const h3_transpose_cfg* cfg, uint32_t launch_rows, uint32_t rows, h3_view x,
                     h3_view out, h3_stream stream) {
  return transpose_common("transpose_f16", cfg, launch_rows, rows, x, out,
                          reinterpret_cast<hipStream_t>(stream), false);
}

int h3_transpose_qkv_v_f16(const h3_transpose_cfg* cfg, uint32_t launch_rows, uint32_t rows,
                           h3_view x, h3_view out, h3_stream stream) {
  return transpose_common("transpose_qkv_v_f16", cfg, launch_rows, rows, x, out,
                          reinterpret_cast<hipStream_t>(stream), true);
}

int h3_prepare_plain_i8(const h3_prepare_plain_cfg* cfg, uint32_t tokens, h3_view x,
                        h3_view codes, h3_view scales, h3_stream stream) {
  const char* stage = "prepare_plain_i8";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  // kernels/prepare_i8_family.loom:202-206
  if (!in_range(cfg->width, 256, 32768, 256))
    return set_error(H3_ERR_CONFIG, "%s: width %u outside [256, 32768] step 256", stage,
                     cfg->width);
  if (!in_range(cfg->lanes, 32, 1024, 32))
    return set_error(H3_ERR_CONFIG, "%s: lanes %u outside [32, 1024] step 32", stage, cfg->lanes);
  if (!in_range(cfg->out_stride, 256, 65536, 64) || cfg->out_stride < cfg->width)
    return set_error(H3_ERR_CONFIG, "%s: out_stride %u outside [width=%u, 65536] step 64", stage,
                     cfg->out_stride, cfg->width);
  if (cfg->elem != H3_ELEM_F16 && cfg->elem != H3_ELEM_BF16 && cfg->elem != H3_ELEM_F32)
    return set_error(H3_ERR_CONFIG, "%s: unknown element format %u", stage, cfg->elem);
  if (!in_range(tokens, 1, 1048576))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 1048576]", stage, tokens);
  const size_t esize = cfg->elem == H3_ELEM_F32 ? 4 : 2;
  h3_view views[3] = {x, codes, scales};
  size_t need[3] = {(size_t)tokens * cfg->width * esize, (size_t)tokens * cfg->out_stride,
                    (size_t)tokens * 4};
  int st = check_bindings(stage, views, need, 3);
  if (st) return st;
  if (reinterpret_cast<uintptr_t>(x.ptr) % 16 || reinterpret_cast<uintptr_t>(codes.ptr) % 16)
    return set_error(H3_ERR_ARGUMENT, "%s: x and codes must be 16-byte aligned", stage);
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_prepare_plain(cfg->width, cfg->out_stride, cfg->elem, tokens,
                                              x.ptr, static_cast<uint8_t*>(codes.ptr),
                                              static_cast<float*>(scales.ptr),
                                              reinterpret_cast<hipStream_t>(stream)));
}

int h3_gemm_i8_qkv_256(const h3_gemm_cfg* cfg, uint32_t tokens, h3_view a, h3_view w,
                       h3_view w_scale, h3_view a_scale, h3_view out, h3_stream stream) {
  const char* stage = "gemm_i8_qkv_256";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  // kernels/gemm_packed_256.loom:3432-3440
  if (!in_range(cfg->k_size, 64, 65536, 64))
    return set_error(H3_ERR_CONFIG, "%s: k_size %u outside [64, 65536] step 64", stage,
                     cfg->k_size);
  if (!in_range(cfg->n_size, 384, 65536, 384))
    return set_error(H3_ERR_CONFIG, "%s: n_size %u outside [384, 65536] step 384", stage,
                     cfg->n_size);
  if (!in_range(cfg->k_stride, 64, 65536, 64) || cfg->k_stride < cfg->k_size)
    return set_error(H3_ERR_CONFIG, "%s: k_stride %u outside [k_size=%u, 65536] step 64", stage,
                     cfg->k_stride, cfg->k_size);
  if (!in_range(cfg->m_group, 1, 4))
    return set_error(H3_ERR_CONFIG, "%s: m_group %u outside [1, 4]", stage, cfg->m_group);
  if (!in_range(tokens, 1, 16777216))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 16777216]", stage, tokens);
  // src/dispatch.rs:1025-1045: the V^T tail is padded to the 256-row capacity.
  const size_t t = tokens, n = cfg->n_size, cap = (t + 255) / 256 * 256;
  h3_view views[5] = {a, w, w_scale, a_scale, out};
  size_t need[5] = {t * cfg->k_stride, n * cfg->k_stride, n * 4, t * 4,
                    (t * n + (cap - t) * (n / 3)) * 2};
  int st = check_bindings(stage, views, need, 5);
  if (st) return st;
  if (reinterpret_cast<uintptr_t>(out.ptr) % 8 != 0)
    return set_error(H3_ERR_ARGUMENT, "%s: out is not 8-byte aligned", stage);
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_gemm_i8_qkv(tokens, cfg->n_size, cfg->k_size, cfg->k_stride,
                                            static_cast<const int8_t*>(a.ptr),
                                            static_cast<const int8_t*>(w.ptr),
                                            static_cast<const float*>(w_scale.ptr),
                                            static_cast<const float*>(a_scale.ptr),
                                            static_cast<uint16_t*>(out.ptr),
                                            reinterpret_cast<hipStream_t>(stream)));
}

int h3_attention_i8qkhm(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_stream stream) {
  return attention_common("attention_i8qkhm", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeHeadI8);
}

int h3_attention_i8qk(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                      h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                      h3_stream stream) {
  return attention_common("attention_i8qk", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI8);
}

int h3_attention_i4qk(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                      h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                      h3_stream stream) {
  return attention_common("attention_i4qk", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI4);
}

namespace {
int attention_i4qks(const h3_attention_skip_cfg* cfg, uint32_t token_count, uint32_t heads,
                    h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                    h3_view workspace, h3_stream stream) {
  const char* stage = "attention_i4qks";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  if (!(cfg->skip_tau == cfg->skip_tau) || cfg->skip_tau > 3.0e38f || cfg->skip_tau < -3.0e38f)
    return set_error(H3_ERR_CONFIG, "%s: skip_tau must be finite", stage);
  const h3_attention_cfg base = {cfg->q_stride, cfg->kv_stride, cfg->out_stride, cfg->tokens,
                                 cfg->token_capacity, cfg->scale};
  return attention_common(stage, &base, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI4Skip,
                          cfg->skip_tau, {}, {}, workspace);
}

int null_workspace(const char* stage) {
  return set_error(H3_ERR_ARGUMENT, "%s: null workspace (use the form without _ws)", stage);
}
}  // namespace

int h3_attention_i4qks(const h3_attention_skip_cfg* cfg, uint32_t token_count, uint32_t heads,
                       h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                       h3_stream stream) {
  return attention_i4qks(cfg, token_count, heads, qi, qs, ki, ks, vt, out, {}, stream);
}

size_t h3_scales_workspace_bytes(const h3_attention_cfg* cfg) {
  return cfg ? scales_workspace_bytes(*cfg) : 0;
}

int h3_attention_i8qk_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                         h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                         h3_view workspace, h3_stream stream) {
  if (!workspace.ptr) return null_workspace("attention_i8qk");
  return attention_common("attention_i8qk", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI8, 0.0f, {}, {},
                          workspace);
}

int h3_attention_i4qk_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                         h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                         h3_view workspace, h3_stream stream) {
  if (!workspace.ptr) return null_workspace("attention_i4qk");
  return attention_common("attention_i4qk", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI4, 0.0f, {}, {},
                          workspace);
}

size_t h3_fp6_workspace_bytes(const h3_attention_cfg* cfg) {
  return cfg ? fp6_layout(*cfg).bytes : 0;
}

int h3_attention_i4qk_fp6(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                          h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                          h3_view workspace, h3_stream stream) {
  if (!workspace.ptr) return null_workspace("attention_i4qk_fp6");
  // the conversion moves 16 bytes per access of the codes and of the workspace rows
  if (int st = check_aligned16("attention_i4qk_fp6", {qi, ki, workspace})) return st;
  return attention_common("attention_i4qk_fp6", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI4Fp6, 0.0f, {}, {},
                          workspace);
}

int h3_attention_i4qks_ws(const h3_attention_skip_cfg* cfg, uint32_t token_count, uint32_t heads,
                          h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                          h3_view out, h3_view workspace, h3_stream stream) {
  if (!workspace.ptr) return null_workspace("attention_i4qks");
  return attention_i4qks(cfg, token_count, heads, qi, qs, ki, ks, vt, out, workspace, stream);
}

// ---------------------------------------------------------------- VSA (kernels/vsa_ops.loom)

int h3_vsa_gather(const h3_vsa_cfg* cfg, h3_view src, h3_view x, h3_view y, h3_stream stream) {
  const char* stage = "VSA gather";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, t = cfg->tokens, w = cfg->width;
  h3_view views[3] = {src, x, y};
  size_t need[3] = {n * 4, t * w * 2, n * w * 2};  // src/vsa/device.rs:216-225
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = check_aligned16(stage, {x, y}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_gather(cfg->tokens, cfg->padded, cfg->width,
                                           static_cast<const int32_t*>(src.ptr),
                                           static_cast<const uint16_t*>(x.ptr),
                                           static_cast<uint16_t*>(y.ptr),
                                           reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_scatter(const h3_vsa_cfg* cfg, h3_view inverse, h3_view x, h3_view y,
                   h3_stream stream) {
  const char* stage = "VSA scatter";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, t = cfg->tokens, w = cfg->width;
  h3_view views[3] = {inverse, x, y};
  size_t need[3] = {t * 4, n * w * 2, t * w * 2};  // src/vsa/device.rs:436-445
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = check_aligned16(stage, {x, y}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_scatter(cfg->tokens, cfg->padded, cfg->width,
                                            static_cast<const int32_t*>(inverse.ptr),
                                            static_cast<const uint16_t*>(x.ptr),
                                            static_cast<uint16_t*>(y.ptr),
                                            reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_pool(const h3_vsa_cfg* cfg, h3_view lengths, h3_view x, h3_view means,
                h3_stream stream) {
  const char* stage = "VSA pool";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, b = cfg->blocks, w = cfg->width;
  h3_view views[3] = {lengths, x, means};
  size_t need[3] = {b * 4, n * w * 2, b * w * 4};  // src/vsa/device.rs:227-238
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = check_aligned16(stage, {x, means}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_pool(cfg->blocks, cfg->width,
                                         static_cast<const int32_t*>(lengths.ptr),
                                         static_cast<const uint16_t*>(x.ptr),
                                         static_cast<float*>(means.ptr),
                                         reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_scores(const h3_vsa_cfg* cfg, h3_view qm, h3_view km, h3_view scores,
                  h3_stream stream) {
  const char* stage = "VSA block scores";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t b = cfg->blocks, w = cfg->width, h = cfg->heads;
  h3_view views[3] = {qm, km, scores};
  size_t need[3] = {b * w * 4, b * w * 4, h * b * b * 4};  // src/vsa/device.rs:240-253
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = check_aligned16(stage, {qm, km}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_scores(cfg->blocks, cfg->heads,
                                           static_cast<const float*>(qm.ptr),
                                           static_cast<const float*>(km.ptr),
                                           static_cast<float*>(scores.ptr),
                                           reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_route(const h3_vsa_cfg* cfg, h3_view scores, h3_view routes, h3_stream stream) {
  const char* stage = "VSA route";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t b = cfg->blocks, h = cfg->heads;
  h3_view views[2] = {scores, routes};
  size_t need[2] = {h * b * b * 4, h * b * b * 4};  // src/vsa/device.rs:254-263
  if ((st = check_bindings(stage, views, need, 2))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_route(cfg->blocks, cfg->heads, cfg->prefix, cfg->topk,
                                          static_cast<const float*>(scores.ptr),
                                          static_cast<int32_t*>(routes.ptr),
                                          reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_coarse(const h3_vsa_cfg* cfg, h3_view scores, h3_view vm, h3_view coarse,
                  h3_stream stream) {
  const char* stage = "VSA coarse attention";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t b = cfg->blocks, w = cfg->width, h = cfg->heads;
  h3_view views[3] = {scores, vm, coarse};
  size_t need[3] = {h * b * b * 4, b * w * 4, b * w * 4};  // src/vsa/device.rs:384-398
  if ((st = check_bindings(stage, views, need, 3))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_coarse(cfg->blocks, cfg->heads,
                                           static_cast<const float*>(scores.ptr),
                                           static_cast<const float*>(vm.ptr),
                                           static_cast<float*>(coarse.ptr),
                                           reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_gated_scatter(const h3_vsa_cfg* cfg, h3_view inverse, h3_view fine, h3_view gate,
                         h3_view coarse, h3_view out, h3_stream stream) {
  const char* stage = "VSA gated scatter";
  int st = check_vsa_cfg(stage, cfg);
  if (st) return st;
  const size_t n = cfg->padded, t = cfg->tokens, b = cfg->blocks, w = cfg->width;
  h3_view views[5] = {inverse, fine, gate, coarse, out};
  size_t need[5] = {t * 4, n * w * 2, t * w * 2, b * w * 4, t * w * 2};  // device.rs:399-433
  if ((st = check_bindings(stage, views, need, 5))) return st;
  if ((st = check_aligned16(stage, {fine, gate, coarse, out}))) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_gated_scatter(cfg->tokens, cfg->padded, cfg->width,
                                                  static_cast<const int32_t*>(inverse.ptr),
                                                  static_cast<const uint16_t*>(fine.ptr),
                                                  static_cast<const uint16_t*>(gate.ptr),
                                                  static_cast<const float*>(coarse.ptr),
                                                  static_cast<uint16_t*>(out.ptr),
                                                  reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_kmean(uint32_t width, uint32_t tokens, h3_view x, h3_view mean, h3_stream stream) {
  const char* stage = "VSA statistics";
  // kernels/vsa_kmean.loom:5, 18
  if (!in_range(width, 128, 65536, 128))
    return set_error(H3_ERR_CONFIG, "%s: width %u outside [128, 65536] step 128", stage, width);
  if (!in_range(tokens, 1, 1048576))
    return set_error(H3_ERR_ARGUMENT, "%s: tokens %u outside [1, 1048576]", stage, tokens);
  h3_view views[2] = {x, mean};
  size_t need[2] = {(size_t)tokens * width * 4, (size_t)width * 4};  // device.rs:334-346
  int st = check_bindings(stage, views, need, 2);
  if (st) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_vsa_kmean(tokens, width, static_cast<const float*>(x.ptr),
                                          static_cast<float*>(mean.ptr),
                                          reinterpret_cast<hipStream_t>(stream)));
}

int h3_attention_i8qkhm_cross(const h3_cross_cfg* cfg, h3_view qi, h3_view qs, h3_view ki,
                              h3_view ks, h3_view vt, h3_view key_mask, h3_view out,
                              h3_stream stream) {
  const char* stage = "cross attention";
  if (!cfg) return set_error(H3_ERR_ARGUMENT, "%s: null config", stage);
  if (!in_range(cfg->q_heads, 1, 256) || !in_range(cfg->kv_heads, 1, 256) ||
      cfg->q_heads % cfg->kv_heads != 0)
    return set_error(H3_ERR_CONFIG, "%s: kv_heads %u must divide q_heads %u (both in [1, 256])",
                     stage, cfg->kv_heads, cfg->q_heads);
  if (!in_range(cfg->q_tokens, 1, 1048576) || !in_range(cfg->kv_tokens, 1, 1048576))
    return set_error(H3_ERR_CONFIG, "%s: q_tokens %u / kv_tokens %u outside [1, 1048576]", stage,
                     cfg->q_tokens, cfg->kv_tokens);
  if (!in_range(cfg->q_capacity, 32, 1048576, 32) || cfg->q_capacity < cfg->q_tokens ||
      !in_range(cfg->kv_capacity, 32, 1048576, 32) || cfg->kv_capacity < cfg->kv_tokens)
    return set_error(H3_ERR_CONFIG,
                     "%s: capacities %u / %u must be multiples of 32 covering the tokens", stage,
                     cfg->q_capacity, cfg->kv_capacity);
  if (!in_range(cfg->out_stride, 128, 32768, 128) || cfg->out_stride < 128 * cfg->q_heads)
    return set_error(H3_ERR_CONFIG, "%s: out_stride %u outside [128 * q_heads, 32768] step 128",
                     stage, cfg->out_stride);
  const size_t qh = cfg->q_heads, kh = cfg->kv_heads, qc = cfg->q_capacity, kc = cfg->kv_capacity;
  h3_view views[7] = {qi, qs, ki, ks, vt, key_mask, out};
  size_t need[7] = {qh * qc * 128, qh * qc * 4, kh * kc * 128, kh * kc * 4, kh * 128 * kc * 2,
                    cfg->kv_tokens, (size_t)cfg->q_tokens * cfg->out_stride * 2};
  int st = check_bindings(stage, views, need, 7);
  if (st) return st;
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_attention_cross(*cfg, static_cast<const int32_t*>(qi.ptr),
                                                static_cast<const float*>(qs.ptr),
                                                static_cast<const int32_t*>(ki.ptr),
                                                static_cast<const float*>(ks.ptr),
                                                static_cast<const uint16_t*>(vt.ptr),
                                                static_cast<const uint8_t*>(key_mask.ptr),
                                                static_cast<uint16_t*>(out.ptr),
                                                reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_attention_i8(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                        h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt, h3_view out,
                        h3_view routes, h3_view lengths, h3_stream stream) {
  return attention_common("VSA attention", cfg, token_count, heads, qi, qs, ki, ks, vt, out,
                          reinterpret_cast<hipStream_t>(stream), kModeTokenI8Vsa, 0.0f, routes,
                          lengths);
}

int h3_vsa_attention_f16(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                         h3_view q, h3_view k, h3_view v, h3_view out, h3_view routes,
                         h3_view lengths, h3_stream stream) {
  const char* stage = "VSA attention f16";
  int st = check_attention_cfg(stage, cfg, token_count, heads);
  if (st) return st;
  // kernels/vsa_attention_16.loom:113-123, 584-587: blocks = tokens / 64 query cubes, routes
  // [out_stride/128][blocks][blocks] i32, lengths [blocks] i32; q [token_capacity][q_stride],
  // k and v [token_capacity][kv_stride], out [token_count][out_stride], all f16.
  if (cfg->tokens % 64 != 0 || cfg->tokens / 64 > 16384)
    return set_error(H3_ERR_CONFIG, "%s: tokens %u is not 64 * blocks with blocks <= 16384",
                     stage, cfg->tokens);
  const size_t cap = cfg->token_capacity, blocks = cfg->tokens / 64;
  const TouchedHeads th = touched_heads(*cfg, heads);
  if (th.q > cfg->q_stride / 128)
    return set_error(H3_ERR_CONFIG, "%s: q_stride %u holds %u query heads, the launch reads %zu",
                     stage, cfg->q_stride, cfg->q_stride / 128, th.q);
  h3_view views[6] = {q, k, v, out, routes, lengths};
  size_t need[6] = {cap * cfg->q_stride * 2,
                    cap * cfg->kv_stride * 2,
                    cap * cfg->kv_stride * 2,
                    ((size_t)(token_count - 1) * cfg->out_stride + th.q * 128) * 2,
                    th.q * blocks * blocks * 4,
                    blocks * 4};
  if ((st = check_bindings(stage, views, need, 6))) return st;
  if ((st = check_aligned16(stage, {q, k, v}))) return st;  // 16-byte row loads
  if ((st = device_ready(stage))) return st;
  return launched(stage, launch_attention_vsa_f16(
                             *cfg, token_count, heads, static_cast<const uint16_t*>(q.ptr),
                             static_cast<const uint16_t*>(k.ptr),
                             static_cast<const uint16_t*>(v.ptr), static_cast<uint16_t*>(out.ptr),
                             static_cast<const int32_t*>(routes.ptr),
                             static_cast<const int32_t*>(lengths.ptr),
                             reinterpret_cast<hipStream_t>(stream)));
}

int h3_vsa_attention_i8_ws(const h3_attention_cfg* cfg, uint32_t token_count, uint32_t heads,
                           h3_view qi, h3_view qs, h3_view ki, h3_view ks, h3_view vt,
                           h3_view out, h3_view routes, h3_view lengths, h3_view workspace,
                           h3_stream stream) {
  if (!workspace.ptr) return null_workspace("VSA attention");
  return vsa_attention_i8_ws(cfg, token_count, heads, qi, qs, ki, ks, vt, out, routes, lengths,
                             workspace, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
