// Host mirror of the reference's INT8 attention block plumbing (src/stack.rs): route selection
// and kernel configs from Stack::build (299-302, 532-766), the IntQk operand bundle
// (229-238, 845-908), Stack::attend (1669-1839) and Stack::prepare_fused_operands (1541-1616).
// Every launch goes through the checked C entry points of abi.cpp, with the byte lengths the
// reference passes as `required`, so an undersized caller buffer fails before any launch.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "internal.hpp"

namespace h3 {
namespace {

// compile::num (src/compile.rs:38-83) spells floats as %.17g; the kernel parses that text as f32.
float config_f32(double v) {
  char buf[64];
  snprintf(buf, sizeof buf, "%.17g", v);
  return strtof(buf, nullptr);
}

// gemm_pitch(k, 16) (src/model.rs:74-85): a 16-bit row whose bytes are a multiple of 1024 is
// padded by 128 elements, so the GEMM's row stride avoids the same-channel conflicts.
uint32_t gemm_pitch16(uint32_t k) { return (2 * k) % 1024 == 0 ? k + 128 : k; }

}  // namespace
}  // namespace h3

struct h3_stack {
  h3_stack_dims d;
  uint32_t capacity = 0;
  uint32_t waves = 0;
  bool head_major = false;   // waves == 8: head-major operands (src/stack.rs:585)
  bool fused = false;        // fused RoPE+quantize operands (src/stack.rs:534-544)
  bool smooth = false;       // K-mean smoothing (H3_KSMOOTH, src/stack.rs:1727-1740)
  h3_prepare_cfg prep_q{}, prep_k{};
  h3_attention_cfg attention{};
  h3_transpose_cfg transpose{};
  // IntQk (src/stack.rs:229-238)
  h3_view qi{}, ki{}, qs{}, ks{}, kmean{}, zmean{}, vt{};
  // The fused route's three independent prepare launches run as branches (the reference
  // records prep_q, prep_k and the V transpose as separate graph branches joined before the
  // attention, src/stack.rs:1751-1813): two side streams at the default priority, forked from
  // and joined back into the caller's stream with events, so the pattern is stream-ordered and
  // capturable.
  hipStream_t side[2] = {nullptr, nullptr};
  hipEvent_t fork = nullptr, join[2] = {nullptr, nullptr};
};

namespace h3 {
namespace {

void release(h3_stack* s) {
  for (h3_view* v : {&s->qi, &s->ki, &s->qs, &s->ks, &s->kmean, &s->zmean, &s->vt})
    if (v->ptr) (void)hipFree(v->ptr);
  for (hipStream_t& st : s->side)
    if (st) (void)hipStreamDestroy(st);
  for (hipEvent_t* e : {&s->fork, &s->join[0], &s->join[1]})
    if (*e) (void)hipEventDestroy(*e);
}

// Branch b of the fused route waits for everything the caller enqueued before the call.
int fork_branches(h3_stack* s, hipStream_t caller) {
  hipError_t e = hipEventRecord(s->fork, caller);
  for (int b = 0; b < 2 && e == hipSuccess; ++b) e = hipStreamWaitEvent(s->side[b], s->fork, 0);
  if (e != hipSuccess)
    return set_error(H3_ERR_LAUNCH, "fused attention operands: forking the branches failed (%s)",
                     hipGetErrorString(e));
  return H3_OK;
}

// The caller's stream waits for both branches (also after a failed launch, so no branch is left
// outside the caller's order).
int join_branches(h3_stack* s, hipStream_t caller) {
  hipError_t e = hipSuccess;
  for (int b = 0; b < 2; ++b) {
    hipError_t r = hipEventRecord(s->join[b], s->side[b]);
    if (r == hipSuccess) r = hipStreamWaitEvent(caller, s->join[b], 0);
    if (e == hipSuccess) e = r;
  }
  if (e != hipSuccess)
    return set_error(H3_ERR_LAUNCH, "fused attention operands: joining the branches failed (%s)",
                     hipGetErrorString(e));
  return H3_OK;
}

}  // namespace
}  // namespace h3

using namespace h3;

extern "C" {

uint32_t h3_capacity(uint32_t tokens, int causal) {
  // src/stack.rs:299-302
  const uint64_t t = tokens;
  const uint64_t waves = (causal || tokens >= 4096) ? 8 : 4;
  uint64_t cap = (t + 16 + 31) / 32 * 32;
  const uint64_t block = 16 * waves;
  cap = std::max(cap, (t + block - 1) / block * block);
  cap = std::max(cap, (t + 255) / 256 * 256);
  return (uint32_t)cap;
}

int h3_stack_build(const h3_stack_dims* dims, h3_stack** out) {
  if (!dims || !out) return set_error(H3_ERR_ARGUMENT, "stack: null argument");
  *out = nullptr;
  if (dims->heads < 1 || dims->heads > 255 || dims->tokens < 1 || dims->tokens > 1048576 ||
      dims->elem > H3_ELEM_BF16)
    return set_error(H3_ERR_ARGUMENT, "stack: heads %u / tokens %u / elem %u out of range",
                     dims->heads, dims->tokens, dims->elem);
  h3_stack* s = new h3_stack();
  s->d = *dims;
  const uint32_t t = dims->tokens, heads = dims->heads, inner = heads * 128;
  s->waves = t >= 4096 ? 8 : 4;
  s->capacity = h3_capacity(t, 0);
  s->head_major = s->waves == 8;
  s->smooth = dims->ksmooth != 0;
  // src/stack.rs:534-544 (plus this build's fused smoothing route when both are asked for)
  s->fused = dims->fused != 0 && s->waves == 8;
  const double extra_q = 1.0 / std::sqrt(128.0) / 128.0;  // src/stack.rs:622-625
  s->prep_q.row_stride = s->fused ? 3 * inner : inner;
  s->prep_q.head_offset = 0;
  s->prep_q.heads = heads;
  s->prep_q.extra_scale = config_f32(extra_q);
  s->prep_q.token_capacity = s->head_major ? s->capacity : 0;
  s->prep_q.eps = config_f32(dims->eps);
  s->prep_q.elem = dims->elem;
  s->prep_k = s->prep_q;
  s->prep_k.extra_scale = 1.0f;  // "the K operand differs only in its head offset" (626-632)
  if (s->fused) s->prep_k.head_offset = inner;
  // src/stack.rs:745-766 (out_stride: the padded pitch on the direct-attention route)
  s->attention.q_stride = inner;
  s->attention.kv_stride = inner;
  s->attention.out_stride = dims->direct_attn ? gemm_pitch16(inner) : inner;
  s->attention.tokens = t;
  s->attention.token_capacity = s->capacity;
  s->attention.scale = config_f32(1.0 / std::sqrt(128.0));
  s->transpose.width = inner;
  s->transpose.row_capacity = s->capacity;
  s->transpose.elem = dims->elem;
  // IntQk buffers, zero-filled once (src/stack.rs:845-908, 889-896)
  const size_t cap = s->capacity;
  struct {
    h3_view* v;
    size_t bytes;
  } allocs[] = {{&s->qi, cap * inner}, {&s->ki, cap * inner},     {&s->qs, cap * heads * 4},
                {&s->ks, cap * heads * 4}, {&s->kmean, inner * 4u}, {&s->zmean, inner * 4u},
                {&s->vt, (size_t)inner * cap * 2}};
  for (auto& a : allocs) {
    if (hipMalloc(&a.v->ptr, a.bytes) != hipSuccess) {
      a.v->ptr = nullptr;  // nothing to free for this one; release() frees the others
      release(s);
      delete s;
      return set_error(H3_ERR_NO_DEVICE, "stack: allocating %zu bytes failed", a.bytes);
    }
    a.v->bytes = a.bytes;
    if (hipMemset(a.v->ptr, 0, a.bytes) != hipSuccess) {  // release() frees it with the others
      release(s);
      delete s;
      return set_error(H3_ERR_NO_DEVICE, "stack: clearing %zu bytes failed", a.bytes);
    }
  }
  if (s->fused) {
    bool ok = true;
    for (hipStream_t& st : s->side)
      ok = ok && hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess;
    for (hipEvent_t* e : {&s->fork, &s->join[0], &s->join[1]})
      ok = ok && hipEventCreateWithFlags(e, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      release(s);
      delete s;
      return set_error(H3_ERR_NO_DEVICE, "stack: creating the branch streams and events failed");
    }
  }
  *out = s;
  return H3_OK;
}

void h3_stack_destroy(h3_stack* stack) {
  if (!stack) return;
  release(stack);
  delete stack;
}

uint32_t h3_stack_capacity(const h3_stack* stack) { return stack ? stack->capacity : 0; }

int h3_stack_operands(const h3_stack* s, h3_int_qk* out) {
  if (!s || !out) return H3_ERR_ARGUMENT;
  out->qi = s->qi;
  out->ki = s->ki;
  out->qs = s->qs;
  out->ks = s->ks;
  out->kmean = s->kmean;
  out->zmean = s->zmean;
  out->vt = s->vt;
  out->head_major = s->head_major ? 1 : 0;
  return H3_OK;
}

static int stack_attention(h3_stack* s, uint32_t t, h3_view out, h3_stream stream) {
  // src/stack.rs:1815-1838: workload [t, heads], scalars [t]
  if (s->head_major)
    return h3_attention_i8qkhm(&s->attention, t, s->d.heads, s->qi, s->qs, s->ki, s->ks, s->vt,
                               out, stream);
  return h3_attention_i8qk(&s->attention, t, s->d.heads, s->qi, s->qs, s->ki, s->ks, s->vt, out,
                           stream);
}

// "the required byte lengths of the reference's emit": a view shorter than `need` is refused.
static int require(const char* stage, int index, h3_view v, size_t need) {
  if (v.bytes < need)
    return set_error(H3_ERR_BINDING, "%s: binding %d is %zu bytes, the kernel addresses %zu",
                     stage, index, v.bytes, need);
  return H3_OK;
}

int h3_stack_attend_fused(h3_stack* s, uint32_t t, h3_view fused, h3_view qnorm, h3_view knorm,
                          h3_view cos_t, h3_view sin_t, h3_view out, h3_stream stream) {
  if (!s) return set_error(H3_ERR_ARGUMENT, "attention: null stack");
  if (!s->fused) return set_error(H3_ERR_ARGUMENT, "fused operands require the fused route");
  if (t < 1 || t > s->d.tokens)
    return set_error(H3_ERR_ARGUMENT, "attention: t %u outside [1, %u]", t, s->d.tokens);
  const size_t rows = t, inner = (size_t)s->d.heads * 128, qkv = 3 * inner;
  const char* stage = "fused attention operands";
  int st;
  // src/stack.rs:1587-1594
  if ((st = require(stage, 0, fused, rows * qkv * 2)) || (st = require(stage, 1, qnorm, 128 * 4)) ||
      (st = require(stage, 1, knorm, 128 * 4)) || (st = require(stage, 2, cos_t, rows * 48 * 4)) ||
      (st = require(stage, 3, sin_t, rows * 48 * 4)) ||
      (st = require("attention", 5, out, rows * s->attention.out_stride * 2)))
    return st;
  // Three branches (src/stack.rs:1751-1813): Q on the caller's stream, K and the V transpose on
  // the side streams, all joined before the attention.
  hipStream_t caller = reinterpret_cast<hipStream_t>(stream);
  if ((st = fork_branches(s, caller))) return st;
  h3_stream k_branch = reinterpret_cast<h3_stream>(s->side[0]);
  h3_stream v_branch = reinterpret_cast<h3_stream>(s->side[1]);
  st = h3_prepare_qk_rope_i8hm(&s->prep_q, t, fused, qnorm, cos_t, sin_t, s->qi, s->qs, stream);
  if (!st) {
    if (s->smooth)
      st = h3_prepare_k_rope_smooth_i8hm(&s->prep_k, t, fused, knorm, cos_t, sin_t, s->kmean,
                                         s->ki, s->ks, k_branch);
    else
      st = h3_prepare_qk_rope_i8hm(&s->prep_k, t, fused, knorm, cos_t, sin_t, s->ki, s->ks,
                                   k_branch);
  }
  // "fused V transpose" (src/stack.rs:1599-1610): workload [t]
  if (!st) st = h3_transpose_qkv_v_f16(&s->transpose, t, t, fused, s->vt, v_branch);
  const int joined = join_branches(s, caller);
  if (st) return st;
  if (joined) return joined;
  return stack_attention(s, t, out, stream);
}

int h3_stack_attend_compact(h3_stack* s, uint32_t t, h3_view compact, h3_view qnorm,
                            h3_view knorm, h3_view cos_t, h3_view sin_t, h3_view out,
                            h3_stream stream) {
  if (!s) return set_error(H3_ERR_ARGUMENT, "attention: null stack");
  // src/stack.rs:634-642: the compact route needs the fused operands and a capacity equal to
  // the 256-row cover the projection writes V^T with.
  const uint32_t tokens = s->d.tokens;
  if (!s->fused || s->capacity != (tokens + 255) / 256 * 256)
    return set_error(H3_ERR_ARGUMENT,
                     "compact operands need the fused route and capacity == ceil(tokens/256)*256 "
                     "(capacity %u, tokens %u)", s->capacity, tokens);
  // V^T sits after the Q/K rows of the stack's token count (src/stack.rs:1034-1040), where the
  // projection of those tokens wrote it.
  if (t != tokens)
    return set_error(H3_ERR_ARGUMENT, "compact operands: t %u must equal the stack's tokens %u", t,
                     tokens);
  const size_t rows = t, inner = (size_t)s->d.heads * 128;
  const size_t vt_offset = rows * 2 * inner * 2, vt_bytes = inner * s->capacity * 2;
  const char* stage = "fused attention operands";
  int st;
  if ((st = require(stage, 0, compact, vt_offset + vt_bytes)) ||
      (st = require("attention", 5, out, rows * s->attention.out_stride * 2)))
    return st;
  // src/stack.rs:643-648: Q/K rows of 2*inner elements, f16 (the projection's output)
  h3_prepare_cfg pq = s->prep_q, pk = s->prep_k;
  pq.row_stride = pk.row_stride = (uint32_t)(2 * inner);
  pq.elem = pk.elem = H3_ELEM_F16;
  h3_view qk = {compact.ptr, vt_offset};
  if ((st = h3_prepare_qk_rope_i8hm(&pq, t, qk, qnorm, cos_t, sin_t, s->qi, s->qs, stream)))
    return st;
  if (s->smooth)
    st = h3_prepare_k_rope_smooth_i8hm(&pk, t, qk, knorm, cos_t, sin_t, s->kmean, s->ki, s->ks,
                                       stream);
  else
    st = h3_prepare_qk_rope_i8hm(&pk, t, qk, knorm, cos_t, sin_t, s->ki, s->ks, stream);
  if (st) return st;
  // No transpose: the projection already wrote V^T (src/stack.rs:1596-1598).
  const h3_view vt = {static_cast<char*>(compact.ptr) + vt_offset, vt_bytes};
  return h3_attention_i8qkhm(&s->attention, t, s->d.heads, s->qi, s->qs, s->ki, s->ks, vt, out,
                             stream);
}

int h3_stack_attend(h3_stack* s, uint32_t t, h3_view q, h3_view k, h3_view v, h3_view out,
                    h3_stream stream) {
  if (!s) return set_error(H3_ERR_ARGUMENT, "attention: null stack");
  if (t < 1 || t > s->d.tokens)
    return set_error(H3_ERR_ARGUMENT, "attention: t %u outside [1, %u]", t, s->d.tokens);
  const size_t rows = t, inner = (size_t)s->d.heads * 128;
  int st;
  if ((st = require("attention operands", 0, q, rows * inner * 2)) ||
      (st = require("attention operands", 0, k, rows * inner * 2)) ||
      (st = require("attention operands", 0, v, rows * inner * 2)) ||
      (st = require("attention", 5, out, rows * s->attention.out_stride * 2)))
    return st;
  h3_prepare_cfg pq = s->prep_q, pk = s->prep_k;
  pq.row_stride = pk.row_stride = (uint32_t)inner;  // separate Q/K buffers (src/stack.rs:609-612)
  pq.head_offset = pk.head_offset = 0;
  if (s->smooth) {  // src/stack.rs:1727-1740
    if ((st = h3_colmean_f32((uint32_t)inner, s->d.elem, t, k, s->kmean, stream))) return st;
  }
  const h3_view kmean = s->smooth ? s->kmean : s->zmean;
  if (s->head_major) {
    if ((st = h3_prepare_qk_i8hm(&pq, t, q, s->zmean, s->qi, s->qs, stream))) return st;
    if ((st = h3_prepare_qk_i8hm(&pk, t, k, kmean, s->ki, s->ks, stream))) return st;
  } else {
    if ((st = h3_prepare_qk_i8(&pq, t, q, s->zmean, s->qi, s->qs, stream))) return st;
    if ((st = h3_prepare_qk_i8(&pk, t, k, kmean, s->ki, s->ks, stream))) return st;
  }
  // V^T over the whole capacity clears the tail (src/stack.rs:1799-1811)
  if ((st = h3_transpose_f16(&s->transpose, s->capacity, t, v, s->vt, stream))) return st;
  return stack_attention(s, t, out, stream);
}

}  // extern "C"
