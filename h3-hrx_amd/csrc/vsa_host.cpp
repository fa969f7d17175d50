// Host side of the VSA path (reference src/vsa.rs and src/vsa/device.rs): the cube plan, the
// routing budget and sigma window of VsaOptions, and the Runtime that owns the VSA buffers and
// emits the per-layer launch sequence. Every launch goes through the checked C entry points
// (abi.cpp), with the byte lengths the reference passes as `required`.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "internal.hpp"

namespace h3 {
namespace {

constexpr uint32_t kModelBlocks = 50;  // src/model.rs:12 (BLOCKS)

// compile::num (src/compile.rs:38-83) spells floats as %.17g; the kernel parses that text as f32.
float config_f32(double v) {
  char buf[64];
  snprintf(buf, sizeof buf, "%.17g", v);
  return strtof(buf, nullptr);
}

uint32_t ceil4(uint32_t v) { return (v + 3) / 4; }

}  // namespace
}  // namespace h3

struct h3_vsa {
  h3_vsa_cfg cfg{};
  h3_attention_cfg attention{};
  h3_prepare_cfg prep_q{}, prep_k{};
  h3_transpose_cfg transpose{};
  uint32_t layers = 0;
  uint32_t bits = 8;  // the attention's operands: 8 (INT8 QK) or 16 (f16 q, k, v)
  // plan (uploaded) and scratch shared by the layers (src/vsa/device.rs:7-46)
  h3_view src{}, inverse{}, lengths{};
  h3_view q{}, k{}, v{}, qm{}, km{}, vm{}, coarse{}, scores{}, routes{}, out{};
  h3_view qi{}, ki{}, qs{}, ks{}, vt{}, zero{};
  h3_view ws{};  // the sparse attention's head-major copy of the key scales
  std::vector<h3_view> means;  // the previous call's K mean of each layer
};

using namespace h3;

namespace {

void release(h3_vsa* r) {
  for (h3_view* v : {&r->src, &r->inverse, &r->lengths, &r->q, &r->k, &r->v, &r->qm, &r->km,
                     &r->vm, &r->coarse, &r->scores, &r->routes, &r->out, &r->qi, &r->ki, &r->qs,
                     &r->ks, &r->vt, &r->zero, &r->ws})
    if (v->ptr) (void)hipFree(v->ptr);
  for (h3_view& v : r->means)
    if (v.ptr) (void)hipFree(v.ptr);
}

int allocate(h3_view* v, size_t bytes, const void* upload = nullptr) {
  if (hipMalloc(&v->ptr, bytes) != hipSuccess) {
    v->ptr = nullptr;
    return set_error(H3_ERR_NO_DEVICE, "VSA: allocating %zu bytes failed", bytes);
  }
  v->bytes = bytes;
  const hipError_t e = upload ? hipMemcpy(v->ptr, upload, bytes, hipMemcpyHostToDevice)
                              : hipMemset(v->ptr, 0, bytes);
  if (e != hipSuccess)
    return set_error(H3_ERR_NO_DEVICE, "VSA: initialising %zu bytes failed: %s", bytes,
                     hipGetErrorString(e));
  return H3_OK;
}

}  // namespace

extern "C" {

int h3_vsa_plan_blocks(const h3_vsa_segment* segments, uint32_t n_segments, uint32_t nt,
                       uint32_t nh, uint32_t nw, uint32_t* blocks) {
  if (!blocks || (n_segments && !segments)) return set_error(H3_ERR_ARGUMENT, "VSA plan: null argument");
  uint64_t b = 0;
  for (uint32_t s = 0; s < n_segments; ++s) b += (segments[s].rows + 63ull) / 64;
  b += (uint64_t)ceil4(nt) * ceil4(nh) * ceil4(nw);
  if (b > 16384) return set_error(H3_ERR_ARGUMENT, "VSA plan: %llu blocks exceed 16384", (unsigned long long)b);
  *blocks = (uint32_t)b;
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

int h3_vsa_plan(const h3_vsa_segment* segments, uint32_t n_segments, uint32_t seq_len,
                uint32_t nt, uint32_t nh, uint32_t nw, int32_t* src, int32_t* inverse,
                int32_t* lengths, uint32_t* prefix_blocks) {
  uint32_t blocks = 0;
  int st = h3_vsa_plan_blocks(segments, n_segments, nt, nh, nw, &blocks);
  if (st) return st;
  if (!src || !inverse || !lengths || !prefix_blocks)
    return set_error(H3_ERR_ARGUMENT, "VSA plan: null argument");
  const uint64_t video = (uint64_t)nt * nh * nw;
  if (video > seq_len) return set_error(H3_ERR_ARGUMENT, "VSA plan: video rows exceed seq_len");
  // src/vsa.rs:98-106: each prefix segment in 64-row tiles, the last padded with -1
  size_t n = 0, b = 0;
  for (uint32_t s = 0; s < n_segments; ++s) {
    const uint64_t start = segments[s].row0, end = start + segments[s].rows;
    if (end > seq_len) return set_error(H3_ERR_ARGUMENT, "VSA plan: segment %u ends past seq_len", s);
    for (uint64_t row = start; row < end; row += 64) {
      const uint64_t live = end - row < 64 ? end - row : 64;
      lengths[b++] = (int32_t)live;
      for (uint64_t r = 0; r < 64; ++r) src[n++] = r < live ? (int32_t)(row + r) : -1;
    }
  }
  *prefix_blocks = (uint32_t)b;
  // src/vsa.rs:111-130: 4x4x4 cubes of (t, h, w) latent cells, row-major inside a cube
  const uint64_t video0 = seq_len - video;
  for (uint32_t t = 0; t < nt; t += 4)
    for (uint32_t h = 0; h < nh; h += 4)
      for (uint32_t w = 0; w < nw; w += 4) {
        const size_t start = n;
        for (uint32_t tt = t; tt < t + 4 && tt < nt; ++tt)
          for (uint32_t hh = h; hh < h + 4 && hh < nh; ++hh)
            for (uint32_t ww = w; ww < w + 4 && ww < nw; ++ww)
              src[n++] = (int32_t)(video0 + ((uint64_t)tt * nh + hh) * nw + ww);
        lengths[b++] = (int32_t)(n - start);
        while (n < start + 64) src[n++] = -1;
      }
  // src/vsa.rs:131-140: the inverse must cover every row once
  for (uint32_t r = 0; r < seq_len; ++r) inverse[r] = -1;
  for (size_t i = 0; i < n; ++i) {
    if (src[i] < 0) continue;
    if (inverse[src[i]] >= 0)
      return set_error(H3_ERR_ARGUMENT, "VSA plan: row %d is listed twice", src[i]);
    inverse[src[i]] = (int32_t)i;
  }
  for (uint32_t r = 0; r < seq_len; ++r)
    if (inverse[r] < 0)
      return set_error(H3_ERR_ARGUMENT, "VSA layout must cover every live token (row %u)", r);
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

int h3_vsa_validate(const h3_vsa_options* o, uint32_t attention_bits) {
  if (!o) return set_error(H3_ERR_ARGUMENT, "VSA: null options");
  // src/vsa.rs:33-52
  if (!std::isfinite(o->keep_percent) || !(o->keep_percent >= 0.0 && o->keep_percent <= 100.0) ||
      o->keep_percent == 0.0)
    return set_error(H3_ERR_ARGUMENT, "VSA keep_percent must be finite and in (0, 100]");
  if (!std::isfinite(o->start) || !std::isfinite(o->end) || o->start < 0.0 || o->end > 1.0 ||
      o->start > o->end)
    return set_error(H3_ERR_ARGUMENT, "VSA requires 0 <= start <= end <= 1");
  bool bad_block = false;
  for (uint32_t i = 0; i < o->n_dense_blocks; ++i)
    bad_block = bad_block || !o->dense_blocks || o->dense_blocks[i] >= kModelBlocks;
  if (o->min_tokens > (1u << 20) || bad_block)
    return set_error(H3_ERR_ARGUMENT, "VSA token threshold or dense block index is out of range");
  // src/vsa.rs:76-85
  if (attention_bits == 4)
    return set_error(H3_ERR_ARGUMENT, "VSA supports f16 or i8 attention, not i4");
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

uint32_t h3_vsa_topk(double keep_percent, uint32_t nonprefix) {
  // src/vsa.rs:54-59: f64 product, round half to even, then max(1), min(nonprefix - 1)
  const double r = std::nearbyint(keep_percent / 100.0 * (double)nonprefix);
  uint64_t k = r > 0.0 ? (uint64_t)r : 0;  // `as usize` saturates at 0
  if (k < 1) k = 1;
  const uint64_t cap = nonprefix > 0 ? nonprefix - 1 : 0;
  return (uint32_t)(k < cap ? k : cap);
}

const char* h3_vsa_dense_reason(const h3_vsa_options* o, uint32_t tokens, float sigma,
                                double shift) {
  if (!o) return "invalid_options";
  // src/vsa.rs:60-72
  auto threshold = [shift](double percent) {
    const double t = 1.0 - percent;
    return (float)(shift * t / (1.0 + (shift - 1.0) * t));
  };
  if (tokens < o->min_tokens) return "below_min_tokens";
  if (sigma > threshold(o->start) || sigma < threshold(o->end)) return "outside_sigma_window";
  return nullptr;
}

int h3_vsa_build(const int32_t* src, const int32_t* inverse, const int32_t* lengths,
                 uint32_t blocks, uint32_t seq_len, uint32_t prefix_blocks,
                 const h3_vsa_options* options, uint32_t heads, uint32_t layers, h3_vsa** out) {
  return h3_vsa_build_bits(src, inverse, lengths, blocks, seq_len, prefix_blocks, options, heads,
                           8, layers, out);
}

int h3_vsa_build_bits(const int32_t* src, const int32_t* inverse, const int32_t* lengths,
                      uint32_t blocks, uint32_t seq_len, uint32_t prefix_blocks,
                      const h3_vsa_options* options, uint32_t heads, uint32_t bits,
                      uint32_t layers, h3_vsa** out) {
  if (!src || !inverse || !lengths || !options || !out)
    return set_error(H3_ERR_ARGUMENT, "VSA build: null argument");
  *out = nullptr;
  int st = h3_vsa_validate(options, bits);
  if (st) return st;
  // src/vsa/device.rs:86 names the attention vsa_attention_{bits}; the INT8 operands exist only
  // for bits 8 (device.rs:104-158).
  if (bits != 8 && bits != 16)
    return set_error(H3_ERR_ARGUMENT, "VSA build: attention bits %u is neither 8 nor 16", bits);
  if (blocks < 1 || blocks > 16384 || seq_len < 1 || seq_len > 1048576 || prefix_blocks > blocks ||
      heads < 1 || heads > 256 || layers < 1)
    return set_error(H3_ERR_ARGUMENT,
                     "VSA build: blocks %u / seq_len %u / prefix %u / heads %u / layers %u out of "
                     "range", blocks, seq_len, prefix_blocks, heads, layers);
  h3_vsa* r = new h3_vsa();
  const uint32_t n = 64 * blocks, width = 128 * heads;
  // src/vsa/device.rs:63-77
  r->cfg = {seq_len, n, width, blocks, heads, prefix_blocks,
            h3_vsa_topk(options->keep_percent, blocks - prefix_blocks)};
  // device.rs:85-95: tokens = token_capacity = padded, strides = width
  r->attention = {width, width, width, n, n, config_f32(1.0 / std::sqrt(128.0))};
  // device.rs:105-119: token-major prepare_qk_i8, Q with 1/128/sqrt(128), K with 1
  r->prep_q = {width, 0, heads, config_f32(1.0 / 128.0 / std::sqrt(128.0)), 0, 0.0f, H3_ELEM_F16};
  r->prep_k = r->prep_q;
  r->prep_k.extra_scale = 1.0f;
  r->transpose = {width, n, H3_ELEM_F16};  // device.rs:120-128
  r->layers = layers;
  r->bits = bits;
  const size_t nw2 = (size_t)n * width * 2, bw4 = (size_t)blocks * width * 4,
               hbb4 = (size_t)heads * blocks * blocks * 4;
  struct {
    h3_view* v;
    size_t bytes;
    const void* upload;
  } allocs[] = {{&r->src, (size_t)n * 4, src},
                {&r->inverse, (size_t)seq_len * 4, inverse},
                {&r->lengths, (size_t)blocks * 4, lengths},
                {&r->q, nw2, nullptr},
                {&r->k, nw2, nullptr},
                {&r->v, nw2, nullptr},
                {&r->qm, bw4, nullptr},
                {&r->km, bw4, nullptr},
                {&r->vm, bw4, nullptr},
                {&r->coarse, bw4, nullptr},
                {&r->scores, hbb4, nullptr},
                {&r->routes, hbb4, nullptr},
                {&r->out, nw2, nullptr}};
  struct {
    h3_view* v;
    size_t bytes;
  } integer[] = {{&r->qi, (size_t)n * width},
                 {&r->ki, (size_t)n * width},
                 {&r->qs, (size_t)n * heads * 4},
                 {&r->ks, (size_t)n * heads * 4},
                 {&r->vt, nw2},
                 {&r->zero, (size_t)width * 4},
                 {&r->ws, scales_workspace_bytes(r->attention)}};
  for (auto& a : allocs) {
    if ((st = allocate(a.v, a.bytes, a.upload))) {
      release(r);
      delete r;
      return st;
    }
  }
  if (bits == 16) {
    *out = r;
    set_error(H3_OK, "%s", "");
    return H3_OK;
  }
  for (auto& a : integer) {
    if ((st = allocate(a.v, a.bytes))) {
      release(r);
      delete r;
      return st;
    }
  }
  r->means.assign(layers, h3_view{});
  for (h3_view& m : r->means) {
    if ((st = allocate(&m, (size_t)width * 4))) {
      release(r);
      delete r;
      return st;
    }
  }
  *out = r;
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

void h3_vsa_destroy(h3_vsa* r) {
  if (!r) return;
  release(r);
  delete r;
}

int h3_vsa_reset(h3_vsa* r, h3_stream stream) {
  if (!r) return set_error(H3_ERR_ARGUMENT, "VSA reset: null runtime");
  for (h3_view& m : r->means) {
    const hipError_t e = hipMemsetAsync(m.ptr, 0, m.bytes, reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess)
      return set_error(H3_ERR_LAUNCH, "VSA reset: %s", hipGetErrorString(e));
  }
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

int h3_vsa_attend(h3_vsa* r, uint32_t layer, h3_view q, h3_view k, h3_view v, h3_view out,
                  h3_view gate, h3_stream stream) {
  if (!r) return set_error(H3_ERR_ARGUMENT, "VSA: null runtime");
  if (layer >= r->layers)
    return set_error(H3_ERR_ARGUMENT, "VSA: layer %u outside [0, %u)", layer, r->layers);
  const h3_vsa_cfg* c = &r->cfg;
  int st;
  // src/vsa/device.rs:215-238: gather q, k, v into the cube layout, and the block means of q and
  // k (and of v, which a gate reads, 388-398), each mean from the pass that writes its rows: the
  // same rows and means as a gather followed by a pool, without reading the rows back. Without a
  // gate the INT8 attention's v is gathered below, by the pass that writes V^T.
  const bool v_with_vt = r->bits != 16 && !gate.ptr;
  if ((st = vsa_gather_pool(c, r->src, r->lengths, q, r->q, r->qm, stream)) ||
      (st = vsa_gather_pool(c, r->src, r->lengths, k, r->k, r->km, stream)) ||
      (st = gate.ptr    ? vsa_gather_pool(c, r->src, r->lengths, v, r->v, r->vm, stream)
            : v_with_vt ? H3_OK
                        : h3_vsa_gather(c, r->src, v, r->v, stream)))
    return st;
  // 239-261: block scores, routes
  if ((st = h3_vsa_scores(c, r->qm, r->km, r->scores, stream)) ||
      (st = h3_vsa_route(c, r->scores, r->routes, stream)))
    return st;
  if (r->bits == 16) {
    // 362-386: the f16 attention reads the gathered q, k, v as they are
    if ((st = h3_vsa_attention_f16(&r->attention, c->padded, c->heads, r->q, r->k, r->v, r->out,
                                   r->routes, r->lengths, stream)))
      return st;
  } else {
    // 290-333: INT8 operands (K centred on the layer's previous mean), V^T, sparse attention
    h3_view& mean = r->means[layer];
    if ((st = h3_prepare_qk_i8(&r->prep_q, c->padded, r->q, r->zero, r->qi, r->qs, stream)) ||
        (st = h3_prepare_qk_i8(&r->prep_k, c->padded, r->k, mean, r->ki, r->ks, stream)) ||
        (st = v_with_vt ? vsa_gather_transpose(c, r->src, v, r->v, r->vt, stream)
                        : h3_transpose_f16(&r->transpose, c->padded, c->padded, r->v, r->vt,
                                           stream)) ||
        (st = vsa_attention_i8_ws(&r->attention, c->padded, c->heads, r->qi, r->qs, r->ki, r->ks,
                                  r->vt, r->out, r->routes, r->lengths, r->ws,
                                  reinterpret_cast<hipStream_t>(stream))))
      return st;
    // 334-346: this call's mean of the block K means, for the layer's next call
    if ((st = h3_vsa_kmean(c->width, c->blocks, r->km, mean, stream))) return st;
  }
  if (gate.ptr) {
    // 399-434: coarse attention over the value means, gated scatter
    if ((st = h3_vsa_coarse(c, r->scores, r->vm, r->coarse, stream))) return st;
    return h3_vsa_gated_scatter(c, r->inverse, r->out, gate, r->coarse, out, stream);
  }
  // 435-445
  return h3_vsa_scatter(c, r->inverse, r->out, out, stream);
}

int h3_vsa_inspect(const h3_vsa* r, uint32_t layer, h3_vsa_buffers* out) {
  if (!r || !out || layer >= r->layers) return set_error(H3_ERR_ARGUMENT, "VSA inspect: bad argument");
  *out = {r->src, r->inverse, r->lengths, r->q, r->k, r->v, r->qm, r->km, r->scores, r->routes,
          r->qi, r->ki, r->qs, r->ks, r->vt, r->out,
          layer < r->means.size() ? r->means[layer] : h3_view{}, r->cfg, r->attention};
  set_error(H3_OK, "%s", "");
  return H3_OK;
}

}  // extern "C"
