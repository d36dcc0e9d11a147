// A decode serving loop driven through the C ABIs alone (no Python): the host
// allocator appends one token per sequence, the pass goes to the device, and every layer
// stores the new K/V and attends in one launch; the step ends with yx_sync, as a
// native engine would run it (crates/yaxus-model/src/engine/mod.rs:530-551 over
// Model::forward, crates/yaxus-model/src/lib.rs:434-453). Prints one JSON line:
// host time per step (allocator + pass upload), whole-step time, and device time for
// the attention launches alone. A third loop runs each layer as the Rust crate's
// Backend::attention does over a wrapped host backend (crates/yaxus-backend-hip/src/
// lib.rs): the layer's qkv copied to the device, yx_attention_qkv_dev, the output
// copied back (synchronous copies, from and to pageable memory, then through pinned
// staging), against the same layer with device-resident qkv and output: the
// per-layer cost of the host round trip.
//
// Usage: decode_loop [steps] [batch] [context] [layers]
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/yaxus_hip.h"
#include "../../include/yaxus_kv_cache.h"

namespace {

void die(const char* what, const char* msg) {
  std::fprintf(stderr, "%s: %s\n", what, msg);
  std::exit(1);
}
#define HIPCHECK(x) \
  do {              \
    if ((x) != YX_OK) die(#x, yx_last_error()); \
  } while (0)
#define KVCHECK(x) \
  do {             \
    if ((x) != YX_OK) die(#x, yx_cache_last_error()); \
  } while (0)

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v.empty() ? 0.0 : v[v.size() / 2];
}

}  // namespace

int main(int argc, char** argv) {
  const int steps = argc > 1 ? std::atoi(argv[1]) : 20;
  const size_t B = argc > 2 ? std::strtoul(argv[2], nullptr, 10) : 16;
  const size_t ctx_len = argc > 3 ? std::strtoul(argv[3], nullptr, 10) : 4000;
  const size_t layers = argc > 4 ? std::strtoul(argv[4], nullptr, 10) : 24;
  const size_t page = 16, hq = 16, hkv = 4, d = 128;
  const size_t pages = B * ((ctx_len + 3 * steps + 12) / page + 2) + 16;  // tokens of the three loops

  yx_cache* cache = nullptr;
  KVCHECK(yx_cache_create(pages, 1 << 20, page, &cache));
  std::vector<uint64_t> seqs(B);
  for (auto& s : seqs) s = yx_cache_new_seq(cache);
  {
    std::vector<size_t> counts(B, ctx_len);
    std::vector<uint32_t> toks(B * ctx_len, 1);
    KVCHECK(yx_cache_append(cache, B, seqs.data(), counts.data(), toks.data()));
  }

  yx_ctx* ctx = nullptr;
  HIPCHECK(yx_ctx_create(0, &ctx));
  yx_kv* kv = nullptr;
  HIPCHECK(yx_kv_create(ctx, layers, pages, page, hkv, d, YX_DTYPE_F16, &kv));
  const size_t per_arena = pages * yx_kv_page_bytes(kv) / 2;
  for (size_t l = 0; l < layers; ++l)
    for (int part = 0; part < 2; ++part) {
      void* p = nullptr;
      HIPCHECK(yx_kv_layer_ptr(kv, l, part, &p));
      HIPCHECK(yx_fill_normal(ctx, p, per_arena, YX_DTYPE_F16, 0x59415855ull, (2 * l + part) * per_arena));
    }
  void *q, *k, *v, *out;
  HIPCHECK(yx_dev_alloc(ctx, B * hq * d * 4, &q));
  HIPCHECK(yx_dev_alloc(ctx, B * hkv * d * 4, &k));
  HIPCHECK(yx_dev_alloc(ctx, B * hkv * d * 4, &v));
  HIPCHECK(yx_dev_alloc(ctx, B * hq * d * 4, &out));
  HIPCHECK(yx_fill_normal(ctx, q, B * hq * d, YX_DTYPE_F32, 7, 0));
  HIPCHECK(yx_fill_normal(ctx, k, B * hkv * d, YX_DTYPE_F32, 7, 1ull << 32));
  HIPCHECK(yx_fill_normal(ctx, v, B * hkv * d, YX_DTYPE_F32, 7, 2ull << 32));
  HIPCHECK(yx_sync(ctx));

  const float scale = 0.08838834764831845f;  // 1 / sqrt(128)
  std::vector<size_t> ones(B, 1);
  std::vector<uint32_t> tok(B, 2);
  std::vector<uint32_t> ids, pos, slot, pt_off, pg;
  std::vector<size_t> last;
  std::vector<yx_page_copy> copies;
  std::vector<uint32_t> src, dst;
  std::vector<double> host_us, step_us, alloc_us, pass_us, first_us, launch_us;
  std::vector<std::chrono::steady_clock::time_point> tl0;
  using clk = std::chrono::steady_clock;
  for (int it = 0; it < steps + 3; ++it) {
    const auto t0 = clk::now();
    KVCHECK(yx_cache_append(cache, B, seqs.data(), ones.data(), tok.data()));
    copies.resize(yx_cache_pending_copies(cache));
    copies.resize(yx_cache_take_copies(cache, copies.data(), copies.size()));
    if (!copies.empty()) {
      src.clear();
      dst.clear();
      for (const auto& c : copies) {
        src.push_back(c.src);
        dst.push_back(c.dst);
      }
      HIPCHECK(yx_kv_copy_pages(ctx, kv, src.data(), dst.data(), src.size()));
    }
    const size_t rows = yx_cache_pass_rows(cache), np = yx_cache_pass_npages(cache);
    ids.resize(rows);
    pos.resize(rows);
    slot.resize(rows);
    pt_off.resize(rows);
    pg.resize(np);
    last.resize(yx_cache_pass_nitems(cache));
    yx_cache_pass_get(cache, ids.data(), pos.data(), slot.data(), pt_off.data(), pg.data(), last.data());
    const auto ta = clk::now();
    HIPCHECK(yx_pass_begin(ctx, rows, pos.data(), slot.data(), pt_off.data(), pg.data(), np));
    const auto t1 = clk::now();
    for (size_t l = 0; l < layers; ++l) {
      HIPCHECK(yx_attention_append_dev(ctx, kv, l, static_cast<float*>(k), static_cast<float*>(v),
                                       static_cast<float*>(q), static_cast<float*>(out), hq, hkv, 0,
                                       scale));
      if (l == 0) tl0.push_back(clk::now());
    }
    const auto tl = clk::now();
    HIPCHECK(yx_sync(ctx));
    const auto t2 = clk::now();
    if (it >= 3) {
      using us = std::chrono::duration<double, std::micro>;
      alloc_us.push_back(us(ta - t0).count());
      pass_us.push_back(us(t1 - ta).count());
      first_us.push_back(us(tl0.back() - t1).count());
      launch_us.push_back(us(tl - tl0.back()).count());
      host_us.push_back(us(t1 - t0).count());
      step_us.push_back(us(t2 - t0).count());
    }
  }
  // The same steps with the host work of step t + 1 (allocator, pass upload) done while
  // step t's launches run: the pass upload is ordered after them on the stream, and the
  // KV bookkeeping does not need step t's sampled tokens (placeholders here; an engine
  // fills them in for the prefix cache once they are read back).
  auto prepare = [&]() {
    KVCHECK(yx_cache_append(cache, B, seqs.data(), ones.data(), tok.data()));
    copies.resize(yx_cache_pending_copies(cache));
    copies.resize(yx_cache_take_copies(cache, copies.data(), copies.size()));
    if (!copies.empty()) {
      src.clear();
      dst.clear();
      for (const auto& c : copies) {
        src.push_back(c.src);
        dst.push_back(c.dst);
      }
      HIPCHECK(yx_kv_copy_pages(ctx, kv, src.data(), dst.data(), src.size()));
    }
    const size_t rows = yx_cache_pass_rows(cache), np = yx_cache_pass_npages(cache);
    ids.resize(rows);
    pos.resize(rows);
    slot.resize(rows);
    pt_off.resize(rows);
    pg.resize(np);
    last.resize(yx_cache_pass_nitems(cache));
    yx_cache_pass_get(cache, ids.data(), pos.data(), slot.data(), pt_off.data(), pg.data(), last.data());
    HIPCHECK(yx_pass_begin(ctx, rows, pos.data(), slot.data(), pt_off.data(), pg.data(), np));
  };
  std::vector<double> over_us;
  prepare();
  auto tprev = clk::now();
  for (int it = 0; it < steps + 3; ++it) {
    for (size_t l = 0; l < layers; ++l)
      HIPCHECK(yx_attention_append_dev(ctx, kv, l, static_cast<float*>(k), static_cast<float*>(v),
                                       static_cast<float*>(q), static_cast<float*>(out), hq, hkv, 0,
                                       scale));
    prepare();
    HIPCHECK(yx_sync(ctx));
    const auto tn = clk::now();
    if (it >= 3) over_us.push_back(std::chrono::duration<double, std::micro>(tn - tprev).count());
    tprev = tn;
  }

  // The Rust crate's Backend::attention: qkv from host memory, output to host memory.
  const size_t qkv_floats = B * (hq + 2 * hkv) * d, rope_len = ctx_len + 3 * steps + 64;
  void *qkv, *qn, *kn, *rope, *out2;
  HIPCHECK(yx_dev_alloc(ctx, qkv_floats * 4, &qkv));
  HIPCHECK(yx_dev_alloc(ctx, d * 4, &qn));
  HIPCHECK(yx_dev_alloc(ctx, d * 4, &kn));
  HIPCHECK(yx_dev_alloc(ctx, rope_len * d * 4, &rope));
  HIPCHECK(yx_dev_alloc(ctx, B * hq * d * 4, &out2));
  HIPCHECK(yx_fill_normal(ctx, qkv, qkv_floats, YX_DTYPE_F32, 9, 0));
  HIPCHECK(yx_fill_normal(ctx, qn, d, YX_DTYPE_F32, 9, 1ull << 32));
  HIPCHECK(yx_fill_normal(ctx, kn, d, YX_DTYPE_F32, 9, 2ull << 32));
  HIPCHECK(yx_fill_normal(ctx, rope, rope_len * d, YX_DTYPE_F32, 9, 3ull << 32));
  std::vector<float> host_qkv(qkv_floats), host_out(B * hq * d);
  HIPCHECK(yx_memcpy_d2h(ctx, host_qkv.data(), qkv, qkv_floats * 4));
  void *pin_in, *pin_out;
  HIPCHECK(yx_host_alloc(ctx, qkv_floats * 4, &pin_in));
  HIPCHECK(yx_host_alloc(ctx, B * hq * d * 4, &pin_out));
  std::vector<double> rt_layer_us, dev_layer_us, pin_layer_us;
  for (int it = 0; it < steps + 3; ++it) {
    prepare();
    HIPCHECK(yx_sync(ctx));
    for (size_t l = 0; l < layers; ++l) {
      const auto a = clk::now();
      HIPCHECK(yx_memcpy_h2d(ctx, qkv, host_qkv.data(), qkv_floats * 4));
      HIPCHECK(yx_attention_qkv_dev(ctx, kv, l, static_cast<float*>(qkv), static_cast<float*>(qn),
                                    static_cast<float*>(kn), static_cast<float*>(rope), rope_len, 1e-6f,
                                    static_cast<float*>(out2), hq, hkv, 0, scale));
      HIPCHECK(yx_memcpy_d2h(ctx, host_out.data(), out2, B * hq * d * 4));
      const auto b = clk::now();
      HIPCHECK(yx_attention_qkv_dev(ctx, kv, l, static_cast<float*>(qkv), static_cast<float*>(qn),
                                    static_cast<float*>(kn), static_cast<float*>(rope), rope_len, 1e-6f,
                                    static_cast<float*>(out2), hq, hkv, 0, scale));
      HIPCHECK(yx_sync(ctx));
      const auto c = clk::now();
      // The same through pinned staging: the host qkv copied into pinned memory, DMA
      // both ways, the output copied out of it.
      std::memcpy(pin_in, host_qkv.data(), qkv_floats * 4);
      HIPCHECK(yx_memcpy_h2d(ctx, qkv, pin_in, qkv_floats * 4));
      HIPCHECK(yx_attention_qkv_dev(ctx, kv, l, static_cast<float*>(qkv), static_cast<float*>(qn),
                                    static_cast<float*>(kn), static_cast<float*>(rope), rope_len, 1e-6f,
                                    static_cast<float*>(out2), hq, hkv, 0, scale));
      HIPCHECK(yx_memcpy_d2h(ctx, pin_out, out2, B * hq * d * 4));
      std::memcpy(host_out.data(), pin_out, B * hq * d * 4);
      const auto e = clk::now();
      if (it >= 3) {
        rt_layer_us.push_back(std::chrono::duration<double, std::micro>(b - a).count());
        dev_layer_us.push_back(std::chrono::duration<double, std::micro>(c - b).count());
        pin_layer_us.push_back(std::chrono::duration<double, std::micro>(e - c).count());
      }
    }
  }

  float ms = 0;
  HIPCHECK(yx_timer_start(ctx));
  for (size_t l = 0; l < layers; ++l)
    HIPCHECK(yx_attention_append_dev(ctx, kv, l, static_cast<float*>(k), static_cast<float*>(v),
                                     static_cast<float*>(q), static_cast<float*>(out), hq, hkv, 0, scale));
  HIPCHECK(yx_timer_stop(ctx, &ms));
  std::printf("{\"batch\": %zu, \"context\": %zu, \"layers\": %zu, \"host_us_median\": %.1f, "
              "\"allocator_us_median\": %.1f, \"pass_begin_us_median\": %.1f, "
              "\"first_layer_call_us_median\": %.1f, \"other_layer_calls_us_median\": %.1f, "
              "\"step_us_median\": %.1f, \"overlapped_step_us_median\": %.1f, "
              "\"attention_us_all_layers\": %.1f, \"host_roundtrip_layer_us_median\": %.1f, "
              "\"host_roundtrip_pinned_layer_us_median\": %.1f, "
              "\"device_layer_us_median\": %.1f, \"qkv_bytes_h2d\": %zu, \"out_bytes_d2h\": %zu}\n",
              B, ctx_len, layers, median(host_us), median(alloc_us), median(pass_us), median(first_us),
              median(launch_us), median(step_us), median(over_us), ms * 1000.0, median(rt_layer_us),
              median(pin_layer_us), median(dev_layer_us), qkv_floats * 4, B * hq * d * 4);
  for (void* p : {q, k, v, out, qkv, qn, kn, rope, out2}) yx_dev_free(ctx, p);
  yx_host_free(ctx, pin_in);
  yx_host_free(ctx, pin_out);
  yx_kv_destroy(ctx, kv);
  yx_ctx_destroy(ctx);
  yx_cache_destroy(cache);
  return 0;
}
