// The C ABI of the device half (include/yaxus_hip.h): contexts, the paged arena, pass
// metadata, split-K work lists and kernel launches. All device work of a context goes
// on its one stream, in call order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <unordered_set>
#include <vector>

#include "../../include/yaxus_hip.h"
#include "attn_decode.hpp"
#include "attn_prefill.hpp"
#include "attn_prefill_f32.hpp"
#include "kv_kernels.hpp"
#include "qk_rope.hpp"
#include "step_after.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& m) {
  g_err = m;
  return code;
}

// A failed call's error is also taken out of HIP's per-thread last error, so that a
// refused allocation is not reported again by the next launch's hipGetLastError().
#define YX_HIP(call)                                                                    \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess) {                                                             \
      (void)hipGetLastError();                                                          \
      return fail(YX_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(e_));       \
    }                                                                                   \
  } while (0)

// A device buffer that only grows. Growing waits for the stream (the old buffer may
// still be read by queued work) and frees the old allocation; it is refused while the
// stream is being captured into a graph (none of those calls may be captured).
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  uint64_t gen = 0;  // (re)allocations and releases so far: a captured graph's check
  int ensure(size_t bytes, hipStream_t s, bool zero = false) {
    if (bytes <= cap) return YX_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    YX_HIP(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone)
      return fail(YX_ERR_INVALID,
                  "a scratch buffer would have to grow during graph capture: run the call once "
                  "with these sizes before capturing it");
    ++gen;
    size_t n = std::max(bytes, cap * 2);
    n = (n + 255) & ~static_cast<size_t>(255);
    if (p) {
      YX_HIP(hipStreamSynchronize(s));
      YX_HIP(hipFree(p));
      p = nullptr;
      cap = 0;
    }
    YX_HIP(hipMalloc(&p, n));
    if (zero) {
      YX_HIP(hipMemsetAsync(p, 0, n, s));
      YX_HIP(hipStreamSynchronize(s));
    }
    cap = n;
    return YX_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    ++gen;
    p = nullptr;
    cap = 0;
  }
};

// Pinned host staging for metadata uploads. Two of them alternate between passes;
// an event marks the last copy issued from each, so it is reused only once drained.
struct Staging {
  char* host = nullptr;
  size_t cap = 0, used = 0;
  hipEvent_t done = nullptr;
  int reset() {
    if (done) YX_HIP(hipEventSynchronize(done));
    used = 0;
    return YX_OK;
  }
  // Whether `bytes` more fit without growing the buffer.
  bool fits(size_t bytes) const { return used + ((bytes + 255) & ~static_cast<size_t>(255)) <= cap; }
  int upload(void* dev, const void* src, size_t bytes, hipStream_t s) {
    if (bytes == 0) return YX_OK;
    size_t need = used + ((bytes + 255) & ~static_cast<size_t>(255));
    if (need > cap) {
      if (done) YX_HIP(hipEventSynchronize(done));
      if (host) YX_HIP(hipHostFree(host));
      host = nullptr;
      size_t n = std::max(need, std::max(cap * 2, static_cast<size_t>(1) << 16));
      YX_HIP(hipHostMalloc(reinterpret_cast<void**>(&host), n, hipHostMallocDefault));
      cap = n;
      used = 0;
      need = (bytes + 255) & ~static_cast<size_t>(255);
    }
    memcpy(host + used, src, bytes);
    YX_HIP(hipMemcpyAsync(dev, host + used, bytes, hipMemcpyHostToDevice, s));
    if (!done) YX_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    YX_HIP(hipEventRecord(done, s));
    used = need;
    return YX_OK;
  }
  // Room for `bytes` at the start of an empty staging buffer (grown when needed), to be
  // filled by the caller and sent with send(): one copy for many pieces.
  int reserve(size_t bytes, char** out) {
    if (used != 0) return fail(YX_ERR_INVALID, "internal: reserve on a staging buffer in use");
    if (bytes > cap) {
      if (done) YX_HIP(hipEventSynchronize(done));
      if (host) YX_HIP(hipHostFree(host));
      host = nullptr;
      cap = 0;
      const size_t n = std::max(bytes, static_cast<size_t>(1) << 16);
      YX_HIP(hipHostMalloc(reinterpret_cast<void**>(&host), n, hipHostMallocDefault));
      cap = n;
    }
    *out = host;
    return YX_OK;
  }
  int send(void* dev, size_t bytes, hipStream_t s) {
    if (bytes) YX_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, s));
    if (!done) YX_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    YX_HIP(hipEventRecord(done, s));
    used = (bytes + 255) & ~static_cast<size_t>(255);
    return YX_OK;
  }
  void release() {
    if (done) (void)hipEventDestroy(done);
    if (host) (void)hipHostFree(host);
    done = nullptr;
    host = nullptr;
  }
};

// The rows of one sequence in a pass. pt_off: its page table in the pass's host page
// tables; dev_off: in the device's page tables (a region that stays put across passes).
struct Group {
  uint32_t r0, n, pt_off, dev_off;
};

// Copies page-table runs into the device's page tables: run r writes runs[3r + 1]
// entries from data[runs[3r + 2]...] to pages[runs[3r]...].
__global__ __launch_bounds__(256) void page_runs_apply(const uint32_t* __restrict__ runs, uint32_t nruns,
                                                       const uint32_t* __restrict__ data,
                                                       uint32_t* __restrict__ pages) {
  for (uint32_t r = blockIdx.x; r < nruns; r += gridDim.x) {
    const uint32_t dst = runs[3 * r], n = runs[3 * r + 1], src = runs[3 * r + 2];
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) pages[dst + i] = data[src + i];
  }
}

// A split-K work list for one (window, hq, hkv) over the current pass.
struct AttnPlan {
  bool prefill = false;  // MFMA tiles over LDS (many rows per sequence) vs split-K decode
  std::vector<yx::PrefillItem> pitems;
  int nt = 1;
  bool balanced = false;  // one tile, items of at most 4 * kBalQuads blocks: waves share a queue
  bool small_units = false;  // balanced with items of at most 2 * kBalQuads blocks: 2-block units
  bool wide = false;  // 16-row tiles (the wide kernel) instead of 8-row ones
  bool f32 = false;   // the f32-arena kernel
  int pf32_waves = 8;  // f32 prefill tiles: 8 waves (128 logical rows) or 4 (64)
  std::vector<yx::AttnItem> items;
  DevBuf d_items;
  std::vector<yx::SubRef> members;  // member groups of shared prefixes
  DevBuf d_members;
  size_t cascades = 0;              // shared prefixes attended once for their groups
  bool fusable = false;  // the append can run inside the attention kernel
  size_t slots = 0;     // partial slots (per kv head)
  size_t counters = 0;  // arrival counters (per kv head)
  bool uploaded = false;  // dev_items / dev_members hold the lists
  // Where the kernels read the lists: d_items / d_members, or the pass's metadata buffer
  // when the plan was built with the pass (yx_pass_begin).
  const void* dev_items = nullptr;
  const void* dev_members = nullptr;
  size_t item_bytes() const {
    return prefill ? pitems.size() * sizeof(yx::PrefillItem) : items.size() * sizeof(yx::AttnItem);
  }
};

struct Profile {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  double total_ms = 0;
  uint64_t launches = 0;
};

constexpr int kMaxCopiesPerLaunch = 64;
struct CopyList {
  uint32_t src[kMaxCopiesPerLaunch];
  uint32_t dst[kMaxCopiesPerLaunch];
};

__global__ __launch_bounds__(256) void kv_copy_pages_list(CopyList list,
                                                          uint4* const* __restrict__ bases,
                                                          uint32_t page_vec16) {
  uint4* base = bases[blockIdx.y];
  const uint4* s = base + static_cast<size_t>(list.src[blockIdx.x]) * page_vec16;
  uint4* d = base + static_cast<size_t>(list.dst[blockIdx.x]) * page_vec16;
  for (uint32_t i = threadIdx.x; i < page_vec16; i += blockDim.x) d[i] = s[i];
}

// The scratch of the entry point that allocates nothing (yx_attention_append_noalloc):
// one file-scope device array per GPU, held from the library's load until the process
// ends. Its device address is taken once per device (hipGetSymbolAddress, at the first
// context on the device) and used everywhere host code needs the memory: the array's
// name is only a host-side stand-in. Layout: arrival counters (zeroed at set-up, left at
// zero by every completed call), a region for work lists, then the partial maxima/sums
// and the partial outputs, each 256-byte aligned.
constexpr size_t kScratchBytes = size_t{16} << 20;
constexpr size_t kScratchCounterBytes = size_t{1} << 20;
constexpr size_t kScratchListBytes = size_t{2} << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Who used a device's scratch last, and which work lists its list region holds. A
// context's lists stay valid for the pass (epoch) they were built for; a call from
// another context first makes its stream wait for the previous user's stream (an event
// recorded there at the hand-over), so calls on different streams do not overlap on
// the scratch.
using PlanKey = std::tuple<size_t, size_t, size_t, bool, size_t>;  // (window, hq, hkv, f32, page)
struct ScratchOwner {
  const yx_ctx* ctx = nullptr;
  hipStream_t stream = nullptr;
  uint64_t epoch = 0;
  size_t list_used = 0;
  std::vector<std::pair<PlanKey, std::pair<size_t, size_t>>> lists;  // key -> (items, members) offsets
  hipEvent_t handover = nullptr;
};
ScratchOwner g_scratch_owner[kMaxDevices];

__global__ void zero_u32(uint32_t* p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// With `device` current: the scratch's address on it (once per device), counters zeroed.
int scratch_init(int device, hipStream_t s) {
  if (device < 0 || device >= kMaxDevices) return fail(YX_ERR_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return YX_OK;
  void* ptr = nullptr;
  YX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (!ptr) return fail(YX_ERR_HIP, "no device address for the scratch array");
  hipLaunchKernelGGL(zero_u32, dim3(16), dim3(256), 0, s, static_cast<uint32_t*>(ptr),
                     static_cast<uint32_t>(kScratchCounterBytes / 4));
  YX_HIP(hipGetLastError());
  YX_HIP(hipStreamSynchronize(s));
  YX_HIP(hipEventCreateWithFlags(&g_scratch_owner[device].handover, hipEventDisableTiming));
  g_scratch_ptr[device] = ptr;
  return YX_OK;
}

// A context that goes away stops being the scratch's owner (its stream is destroyed).
void scratch_forget(const yx_ctx* c, int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchOwner& o = g_scratch_owner[device];
  if (o.ctx == c) {
    o.ctx = nullptr;
    o.stream = nullptr;
    o.lists.clear();
    o.list_used = 0;
  }
}

struct ScratchMap {
  void *counters, *items, *members, *part_ml, *part_o;
};

}  // namespace

struct yx_kv {
  size_t layers, pages, page, hkv, d;
  bool f32 = false;  // f32 K/V (K in V's layout) instead of binary16
  std::vector<_Float16*> k, v;  // per layer; float* when f32
  DevBuf bases;  // 2 * layers pointers for the copy kernel
  size_t page_bytes() const { return hkv * page * d * (f32 ? 4 : 2); }
  float* kf(size_t l) const { return reinterpret_cast<float*>(k[l]); }
  float* vf(size_t l) const { return reinterpret_cast<float*>(v[l]); }
};

struct yx_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  Staging staging[2];
  int cur_staging = 0;
  // pass
  size_t rows = 0, npages = 0;
  std::vector<uint32_t> pos, slot, pt_off, pages;
  std::vector<Group> groups;
  uint32_t max_page = 0, max_slot = 0;
  // Device pass metadata. d_meta: this pass's positions and slots, the page-table runs
  // that changed since the previous pass, and the work lists built with the pass, sent
  // as one copy. d_pages: the page tables, one region per group that stays put from pass
  // to pass while the groups keep their order and fit (a decode step then sends only the
  // entries that changed: a new page, a copied one).
  DevBuf d_meta, d_pages;
  const uint32_t* dev_pos = nullptr;
  const uint32_t* dev_slot = nullptr;
  std::vector<uint32_t> region_off, region_cap;  // per group of the previous pass
  std::vector<uint32_t> dev_mirror;              // what d_pages holds, entry by entry
  std::vector<std::tuple<size_t, size_t, size_t, bool, size_t>> used_keys;  // plans used this pass
  uint64_t pages_sent = 0, runs_sent = 0;        // page-table entries and runs uploaded (tests)
  uint64_t split_tiles = 0;                       // prefill tiles split along keys (tests)
  uint64_t prefill_plans = 0;                     // work lists built as prefill tiles (tests)
  bool have_pass = false;
  std::map<std::tuple<size_t, size_t, size_t, bool, size_t>, AttnPlan> plans;  // (window, hq, hkv, f32, page)
  // Work-list buffers of dropped plans, reused by the next pass's plans: a new pass
  // uploads into them on the stream, after the launches that read them, so it needs
  // neither a hipFree (which waits for the device) nor a hipMalloc.
  std::vector<DevBuf> spare;
  DevBuf take_spare() {
    if (spare.empty()) return DevBuf{};
    DevBuf b = spare.back();
    spare.pop_back();
    return b;
  }
  // Drops the cached plans (a new pass or option), keeping their device buffers.
  void retire_plans() {
    for (auto& kv : plans)
      for (DevBuf* b : {&kv.second.d_items, &kv.second.d_members})
        if (b->p) {
          spare.push_back(*b);
          *b = DevBuf{};
        }
    plans.clear();
  }
  // scratch
  DevBuf part_o, part_ml, counters, io_a, io_b, io_c, io_q;
  DevBuf am_keys, am_counters;  // argmax: per-slice keys, per-row arrival counters
  DevBuf mm_part, mm_counters;  // matmul: per-k-part output tiles, per-tile arrival counters
  // options
  long target_waves = 0;  // 0: one work item per CU
  int cus = 256;
  long max_chunk_blocks = 1 << 20;
  long prefill_min_rows = 0;  // 0: automatic (see build_plan)
  // Most 8-row units of logical rows per work item. The wide kernel holds 32 rows in two
  // 16-row tiles; the static 8-row-tile kernel spills with a fourth tile, so it keeps 3
  // unless one row's q heads need 4.
  long max_tiles = 4;
  // 0: automatic (the queue or the 16-row-tile kernel), 1: 8-row-tile static split only,
  // 2: the 16-row-tile kernel for every decode pass.
  long decode_shape = 0;
  long cascade = 1;  // attend keys shared by consecutive groups (same pages) once for all of them
  long xcd_prefix = 1;  // place the readers of one shared-prefix chunk on one XCD
  long prefill_split = 1;  // split long prefill tiles along keys when the pass underfills the GPU
  long matmul_k_split = 0;  // workgroups per matmul output tile along k (0: automatic)
  long argmax_slices = 0;   // workgroups per argmax row (0: automatic)
  long pf32_waves = 0;      // f32 prefill tile shape: 4 or 8 waves (0: automatic)
  bool profiling = false;
  Profile prof[4];
  bool capturing = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  // What a captured graph's kernels point at: a new pass, an option, a destroyed arena
  // (epoch) or a reallocated buffer (DevBuf::gen) invalidates it.
  // Work lists are freed only with an epoch step; the other buffers count their own
  // reallocations; both only grow, so the pair changes whenever either does.
  uint64_t epoch = 0, graph_epoch = 0, graph_gens = 0;
  uint64_t buffer_gens() const {
    uint64_t s = 0;
    for (const DevBuf* b : {&d_meta, &d_pages, &part_o, &part_ml, &counters, &io_a, &io_b, &io_c,
                            &io_q, &am_keys, &am_counters, &mm_part, &mm_counters})
      s += b->gen;
    return s;
  }

  int set_device() {
    YX_HIP(hipSetDevice(device));
    return YX_OK;
  }
};

namespace {

// Regions of the device's scratch for one no-alloc call; refuses sizes beyond it.
int scratch_map(yx_ctx* c, size_t part_ml, size_t part_o, size_t counters, ScratchMap* m) {
  char* base = static_cast<char*>(g_scratch_ptr[c->device]);
  if (!base) return fail(YX_ERR_INVALID, "scratch not set up on this device");
  if (counters > kScratchCounterBytes)
    return fail(YX_ERR_UNSUPPORTED, "no-alloc call: the pass needs more arrival counters than the scratch holds");
  auto r256 = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  size_t off = kScratchCounterBytes + kScratchListBytes;
  m->counters = base;
  m->items = m->members = nullptr;
  m->part_ml = base + off;
  off += r256(part_ml);
  m->part_o = base + off;
  off += r256(part_o);
  if (off > kScratchBytes)
    return fail(YX_ERR_UNSUPPORTED, "no-alloc call: the pass's split-K partials need " +
                                        std::to_string(off) + " bytes, more than the " +
                                        std::to_string(kScratchBytes) + "-byte scratch");
  return YX_OK;
}

// Takes the device's scratch for context c: when another context used it last, c's
// stream first waits for everything issued on that context's stream so far (one event,
// no allocation). Under graph capture the wait cannot be recorded, so a hand-over there
// is refused. Then finds the plan's work lists in the scratch's list region, or sends
// them there from the pass's pinned staging (once per plan and pass); plans whose lists
// yx_pass_begin already put on the device are read from there instead.
int scratch_take(yx_ctx* c, const PlanKey& key, AttnPlan* plan, ScratchMap* m) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchOwner& o = g_scratch_owner[c->device];
  if (o.ctx != c) {
    if (o.ctx) {
      if (c->capturing)
        return fail(YX_ERR_INVALID, "no-alloc call under capture: another context used this GPU's scratch last; "
                                    "make one eager call first");
      YX_HIP(hipEventRecord(o.handover, o.stream));
      YX_HIP(hipStreamWaitEvent(c->stream, o.handover, 0));
    }
    o.ctx = c;
    o.stream = c->stream;
    o.lists.clear();
    o.list_used = 0;
  }
  if (plan->uploaded) {
    m->items = const_cast<void*>(plan->dev_items);
    m->members = const_cast<void*>(plan->dev_members);
    return YX_OK;
  }
  if (o.epoch != c->epoch) {
    o.epoch = c->epoch;
    o.lists.clear();
    o.list_used = 0;
  }
  char* base = static_cast<char*>(g_scratch_ptr[c->device]) + kScratchCounterBytes;
  for (const auto& e : o.lists)
    if (e.first == key) {
      m->items = base + e.second.first;
      m->members = base + e.second.second;
      return YX_OK;
    }
  auto r256 = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  const size_t ib = plan->item_bytes(), mb = plan->members.size() * sizeof(yx::SubRef);
  if (c->capturing)
    return fail(YX_ERR_INVALID, "run the call once before capturing it (its work list is uploaded then)");
  if (o.list_used + r256(ib) + r256(mb) > kScratchListBytes)
    return fail(YX_ERR_UNSUPPORTED, "no-alloc call: the pass's work lists need more than the scratch's " +
                                        std::to_string(kScratchListBytes) + "-byte list region");
  Staging& st = c->staging[c->cur_staging];
  if (!st.fits(r256(ib) + r256(mb)))
    return fail(YX_ERR_UNSUPPORTED, "work list larger than the pass's staging buffer (no-alloc call)");
  const size_t oi = o.list_used, om = oi + r256(ib);
  const void* items = plan->prefill ? static_cast<const void*>(plan->pitems.data()) : plan->items.data();
  int rc;
  if ((rc = st.upload(base + oi, items, ib, c->stream))) return rc;
  if (mb && (rc = st.upload(base + om, plan->members.data(), mb, c->stream))) return rc;
  o.list_used = om + r256(mb);
  o.lists.emplace_back(key, std::make_pair(oi, om));
  m->items = base + oi;
  m->members = base + om;
  return YX_OK;
}

int prof_begin(yx_ctx* c, int which, hipEvent_t* e0) {
  *e0 = nullptr;
  if (!c->profiling) return YX_OK;
  YX_HIP(hipEventCreate(e0));
  YX_HIP(hipEventRecord(*e0, c->stream));
  return YX_OK;
}

int prof_end(yx_ctx* c, int which, hipEvent_t e0) {
  if (!e0) return YX_OK;
  hipEvent_t e1;
  YX_HIP(hipEventCreate(&e1));
  YX_HIP(hipEventRecord(e1, c->stream));
  c->prof[which].pending.emplace_back(e0, e1);
  return YX_OK;
}

int check_kv(yx_ctx* c, yx_kv* kv, size_t layer) {
  if (!c || !kv) return fail(YX_ERR_INVALID, "null context or arena");
  if (layer >= kv->layers) return fail(YX_ERR_INVALID, "layer out of range");
  if (!c->have_pass) return fail(YX_ERR_INVALID, "no pass: call yx_pass_begin first");
  if (c->npages && c->max_page >= kv->pages)
    return fail(YX_ERR_INVALID, "a page table names a page beyond the arena");
  if (c->rows && c->max_slot >= kv->pages * kv->page)
    return fail(YX_ERR_INVALID, "a kv_slot lies beyond the arena");
  // Every key a row can see (up to its position) must have a page-table entry.
  for (size_t i = 0; i < c->rows; ++i)
    if ((c->pos[i] / kv->page) + c->pt_off[i] >= c->npages)
      return fail(YX_ERR_INVALID, "a row's position has no page-table entry");
  return YX_OK;
}

// Builds the split-K work list of the current pass for (window, hq, hkv).
static constexpr uint32_t kFanIn = 32;  // chunks per group the automatic split aims at most

// f32: the f32 arena's plan: its prefill kernel's items for passes with many rows per
// sequence (as for f16), else its split-K decode kernel's (16 logical rows per item).
// page_size: the arena's (shared prefixes are found by page ids).
int build_plan(yx_ctx* c, size_t window, size_t hq, size_t hkv, bool f32, size_t page_size,
               AttnPlan** out) {
  auto key = std::make_tuple(window, hq, hkv, f32, page_size);
  auto it = c->plans.find(key);
  if (it != c->plans.end()) {
    *out = &it->second;
    return YX_OK;
  }
  const size_t G = hq / hkv;
  uint32_t max_rows = 0;
  for (const Group& g : c->groups) max_rows = std::max(max_rows, g.n);
  // Prefill tiles or split-K decode items. With a fixed threshold (option
  // prefill_min_rows > 0), by rows of one sequence. Automatically (0, the default): the
  // prefill kernel when a sequence has more logical rows than one decode work item holds
  // (the decode kernels would read its keys once per item) and the pass makes at least
  // one prefill tile per 8 CUs (with fewer, its tiles split into chunks too short to pay
  // for their merge: one sequence of 32-64 rows after 4096-32768 keys runs 1.2-2x faster
  // as decode items). Measured (B x rows after
  // ctx, decode / prefill us): 16 x 10 after 4096 57.1 / 49.5, 16 x 8 34.2 / 43.0, 1 x 32
  // after 32768 50.1 / 101.1, 1 x 128 after 32768 218.1 / 103.6, 2 x 64 after 16384
  // 81.5 / 70.7.
  bool use_prefill;
  if (c->prefill_min_rows > 0) {
    use_prefill = max_rows >= static_cast<uint32_t>(c->prefill_min_rows);
  } else if (f32) {
    // The f32 arena: its decode items hold 16 logical rows each and re-read their
    // sequence's keys once per item (about 6 TB/s over those reads); its prefill tiles
    // (64 or 128 logical rows, 8 waves per CU) take about 95 us plus 2.4 us per 1024 keys
    // of the longest context (the key split's chain), or 40 us plus their products at
    // 110 TFLOP/s, whichever is more. The kernel with the smaller estimate runs. Measured
    // (B x rows after ctx, decode / prefill us; the choice was right in 19 of 21 shapes,
    // the two misses 5% and 30%): 1 x 32 after 4096 32.6 / 101.8, 1 x 128 after 4096
    // 83.9 / 107.2, 32 x 8 after 2048 94.8 / 119.2, 1 x 48 after 16384 186.6 / 133.4,
    // 1 x 96 after 8192 197.4 / 118.9, 4 x 32 after 8192 177.6 / 129.5, 16 x 10 after
    // 4096 172.0 / 127.6, 1 x 32 after 32768 137.7 / 178.7, 1 x 64 after 32768
    // 453.3 / 217.3, 16 x 256 after 1024 812.5 / 352.8.
    double decode_bytes = 0, flops = 0;
    uint32_t max_keys = 0;
    for (const Group& g : c->groups) {
      uint32_t keys = 0;
      for (uint32_t i = g.r0; i < g.r0 + g.n; ++i) keys = std::max(keys, c->pos[i] + 1);
      if (window > 0) keys = static_cast<uint32_t>(std::min<uint64_t>(keys, window + g.n));
      max_keys = std::max(max_keys, keys);
      decode_bytes += static_cast<double>((g.n * G + 15) / 16) * keys;
      flops += static_cast<double>(g.n) * G * keys;
    }
    decode_bytes *= static_cast<double>(hkv) * yx::kD * sizeof(float) * 2;
    flops *= static_cast<double>(hkv) * 4 * yx::kD;
    const double decode_us = decode_bytes / 6e6;
    const double prefill_us = std::max(95.0 + 2.4 * max_keys / 1024.0, 40.0 + flops / 1.1e8);
    use_prefill = max_rows * G > 16 && decode_us > prefill_us;
  } else {
    size_t tiles = 0;
    for (const Group& g : c->groups) tiles += (g.n * G + yx::kPrefillRows - 1) / yx::kPrefillRows;
    tiles *= hkv;
    use_prefill = max_rows * G > static_cast<size_t>(c->max_tiles) * 8 &&
                  tiles * 8 >= static_cast<size_t>(c->cus);
  }
  if (use_prefill) {
    ++c->prefill_plans;
    // Tiles of kPrefillRows logical rows: consecutive rows of one sequence (the f16 and
    // the f32 arena's prefill kernels take the same items).
    AttnPlan plan;
    plan.prefill = true;
    plan.f32 = f32;
    // f32 tiles of 64 logical rows (two 4-wave workgroups per CU) when every sequence's
    // rows fit one (option prefill_f32_waves: 4 or 8 fixes the shape).
    if (f32)
      plan.pf32_waves = c->pf32_waves ? static_cast<int>(c->pf32_waves)
                                      : (max_rows * G <= static_cast<size_t>(yx::kPf32SmallRows) ? 4 : 8);
    const size_t tile_rows = !f32 ? yx::kPrefillRows : plan.pf32_waves == 4 ? yx::kPf32SmallRows : yx::kPf32Rows;
    const uint32_t per = static_cast<uint32_t>(std::max<size_t>(1, tile_rows / G));
    if (G > tile_rows)
      return fail(YX_ERR_UNSUPPORTED, "more query heads per KV head than a prefill tile holds");
    for (const Group& g : c->groups)
      for (uint32_t r = 0; r < g.n; r += per) {
        yx::PrefillItem w{};
        w.r0 = g.r0 + r;
        w.nrows = std::min(per, g.n - r);
        w.pt_off = g.dev_off;
        uint32_t lo = UINT32_MAX, hi = 0;
        for (uint32_t i = w.r0; i < w.r0 + w.nrows; ++i) {
          const uint32_t p = c->pos[i];
          lo = std::min(lo, (window > 0 && p + 1 > window) ? p + 1 - static_cast<uint32_t>(window) : 0u);
          hi = std::max(hi, p);
        }
        w.blk0 = lo / 16;
        w.blk1 = hi / 16 + 1;
        w.chunk_nch = 1u << 16;
        plan.pitems.push_back(w);
      }
    // Tiles longer than 1.5 times the average load of a workgroup slot (two per CU; a
    // long context with few tiles: one sequence's chunk after thousands of keys) are
    // split along keys into chunks of about that load, at least kMinChunkPairs pairs of
    // blocks each; the chunks' partial results are merged by the tile's last chunk.
    // (cfg3's tiles, 1024 over 512 slots, stay whole.)
    if (c->prefill_split) {
      constexpr uint64_t kFixedPairs = 4;     // a tile's start and output, in pairs
      constexpr uint32_t kMinChunkPairs = 16;
      uint64_t total = 0;
      for (const yx::PrefillItem& w : plan.pitems) total += (w.blk1 - w.blk0 + 1) / 2 + kFixedPairs;
      total *= hkv;
      // Workgroup slots: two per CU (4-wave tiles), one (8-wave f32 tiles).
      const uint64_t slots2 = (f32 && plan.pf32_waves == 8 ? 1 : 2) * static_cast<uint64_t>(c->cus);
      const uint64_t avg = std::max<uint64_t>(kMinChunkPairs, (total + slots2 - 1) / slots2);
      std::vector<yx::PrefillItem> split;
      uint32_t nslot = 0, ncnt = 0;
      for (const yx::PrefillItem& w : plan.pitems) {
        const uint32_t pairs = (w.blk1 - w.blk0 + 1) / 2;
        uint32_t nch = 1;
        if (2 * static_cast<uint64_t>(pairs) > 3 * avg)
          nch = static_cast<uint32_t>(std::min<uint64_t>({(pairs + avg - 1) / avg, pairs / kMinChunkPairs, 64}));
        if (nch <= 1) {
          split.push_back(w);
          continue;
        }
        for (uint32_t ch = 0; ch < nch; ++ch) {
          yx::PrefillItem x = w;
          // Chunk boundaries on pairs of blocks (the kernel's stage unit).
          x.blk0 = w.blk0 + 2 * static_cast<uint32_t>(static_cast<uint64_t>(pairs) * ch / nch);
          x.blk1 = ch + 1 == nch ? w.blk1 : w.blk0 + 2 * static_cast<uint32_t>(static_cast<uint64_t>(pairs) * (ch + 1) / nch);
          x.chunk_nch = (nch << 16) | ch;
          x.part_base = nslot;
          x.counter = ncnt;
          split.push_back(x);
        }
        nslot += nch;
        ++ncnt;
      }
      plan.pitems = std::move(split);
      plan.slots = nslot;
      plan.counters = ncnt;
      c->split_tiles += ncnt;
    }
    // Longest first: the GPU hands work items to CUs in order as they free up, so
    // this bounds the busiest CU near the average (contexts differ a lot in a pass).
    std::stable_sort(plan.pitems.begin(), plan.pitems.end(),
                     [](const yx::PrefillItem& a, const yx::PrefillItem& b) {
                       return a.blk1 - a.blk0 > b.blk1 - b.blk0;
                     });
    auto& p = c->plans[key];
    p = std::move(plan);
    *out = &p;
    return YX_OK;
  }
  size_t nt = (max_rows * G + 7) / 8;
  const long cap = f32 ? 2 : c->decode_shape != 1 ? c->max_tiles : std::min<long>(c->max_tiles, 3);
  nt = std::max<size_t>(1, std::min<size_t>(nt, static_cast<size_t>(cap)));
  nt = std::max<size_t>(nt, (G + 7) / 8);  // one row's q heads always fit one work item
  if (f32 && nt > 2) return fail(YX_ERR_UNSUPPORTED, "f32 arena: more than 16 query heads per KV head");
  const size_t rows_per_sub = nt * 8 / G;
  if (rows_per_sub == 0) return fail(YX_ERR_UNSUPPORTED, "more than 32 query heads per KV head");

  struct Sub {
    uint32_t r0, n, pt_off, dev_off, b0, b1;
    int casc = -1;  // the shared prefix it belongs to
  };
  std::vector<Sub> subs;
  size_t work = 0;
  for (const Group& g : c->groups) {
    for (uint32_t r = 0; r < g.n; r += static_cast<uint32_t>(rows_per_sub)) {
      Sub s;
      s.r0 = g.r0 + r;
      s.n = std::min<uint32_t>(static_cast<uint32_t>(rows_per_sub), g.n - r);
      s.pt_off = g.pt_off;
      s.dev_off = g.dev_off;
      uint32_t lo = UINT32_MAX, hi = 0;
      for (uint32_t i = s.r0; i < s.r0 + s.n; ++i) {
        uint32_t p = c->pos[i];
        uint32_t l = (window > 0 && p + 1 > window) ? p + 1 - static_cast<uint32_t>(window) : 0;
        lo = std::min(lo, l);
        hi = std::max(hi, p);
      }
      s.b0 = lo / 16;
      s.b1 = hi / 16 + 1;
      work += s.b1 - s.b0;
      subs.push_back(s);
    }
  }
  // Shared prefixes (cascade attention): a run of consecutive groups in consecutive pass
  // rows whose page tables start with the same pages reads those keys once, as one
  // group of all their rows (at most 16 logical rows, one tile of the 16-row-tile
  // kernel), instead of once per group. Only keys every row of the run sees (below
  // each row's position, no window cut) are shared; at least kMinShared blocks.
  struct Casc {
    uint32_t r0, n, dev_off, blocks, first, count;
  };
  std::vector<Casc> cascs;
  const uint32_t bpp = static_cast<uint32_t>(page_size / 16);  // blocks per page
  constexpr uint32_t kMinShared = 16;
  if (c->cascade && nt == 1 && c->decode_shape == 0) {
    const uint32_t cap_rows = static_cast<uint32_t>(16 / G);
    for (size_t i = 0; i < subs.size();) {
      size_t j = i + 1;
      uint32_t rows = subs[i].n;
      const uint32_t first_page = c->pages[subs[i].pt_off];
      while (j < subs.size() && subs[j].r0 == subs[j - 1].r0 + subs[j - 1].n &&
             rows + subs[j].n <= cap_rows && subs[j].b0 == 0 && subs[i].b0 == 0 &&
             c->pages[subs[j].pt_off] == first_page)
        rows += subs[j++].n;
      if (j - i >= 2) {
        // Blocks every row sees: below the smallest position's block (so the rows' own
        // new keys are never in the shared part) and within the common pages.
        uint32_t blocks = UINT32_MAX;
        for (size_t k = i; k < j; ++k)
          for (uint32_t r = subs[k].r0; r < subs[k].r0 + subs[k].n; ++r)
            blocks = std::min(blocks, c->pos[r] / 16);
        uint32_t pages_common = (blocks + bpp - 1) / bpp;
        for (size_t k = i + 1; k < j; ++k) {
          uint32_t p = 0;
          while (p < pages_common && c->pages[subs[k].pt_off + p] == c->pages[subs[i].pt_off + p]) ++p;
          pages_common = p;
        }
        blocks = std::min(blocks, pages_common * bpp);
        if (blocks >= kMinShared) {
          Casc cc{subs[i].r0, rows, subs[i].dev_off, blocks, static_cast<uint32_t>(i),
                  static_cast<uint32_t>(j - i)};
          for (size_t k = i; k < j; ++k) {
            work -= blocks;  // read once below, not once per group
            subs[k].b0 = blocks;
            subs[k].casc = static_cast<int>(cascs.size());
          }
          work += blocks;
          cascs.push_back(cc);
        }
      }
      i = j;
    }
  }
  work *= hkv;
  // Work items (workgroups of DecodeWaves waves) aimed at: target_waves / waves.
  // One workgroup per CU runs at a time for every tile count (8 waves of ~220
  // registers, or 4 of more than 256), so by default the split aims at one work item
  // per CU: more would run in a second round.
  // (Four 8-row tiles do not fit one wave's registers: a row with more than 24 q heads
  // per KV head takes the 16-row-tile kernel whatever the shape option.)
  const bool wide = f32 || (nt > 1 && c->decode_shape == 0) || c->decode_shape == 2 || nt > 3;
  const size_t waves = nt == 1 ? yx::DecodeWaves<1>::value
                               : (wide ? yx::kWideWaves : yx::DecodeWaves<2>::value);
  const size_t target_items = c->target_waves > 0
                                  ? std::max<size_t>(1, static_cast<size_t>(c->target_waves) / waves)
                                  : static_cast<size_t>(c->cus);
  size_t cb = (work + target_items - 1) / target_items;
  // At least a unit of blocks per wave (two blocks in the one-tile kernel, whose small
  // items take 2-block units): with less, waves of every work item sit idle and the
  // extra chunks only lengthen the merge (small passes, e.g. sliding windows).
  // Except in tiny passes (at most two blocks per CU, e.g. a few sequences of 512
  // keys): there one quad per work item, at most 8 chunks per group, spreads the loads
  // over more CUs (B=1 ctx 512 9.1 -> 8.4 us, B=4 ctx 512 9.8 -> 8.6).
  const bool tiny = c->target_waves == 0 && nt == 1 && work <= 2 * static_cast<size_t>(c->cus);
  if (c->target_waves == 0 && !tiny) cb = std::max<size_t>(cb, (nt == 1 ? 2 : 4) * waves);
  // Quads per chunk of a group of nq quads for chunks of about cb blocks: at most
  // kMaxChunks chunks, and (automatic split) at most kFanIn chunks per group while
  // chunks stay within the one-tile queue kernel's 16 quads: a few long sequences
  // would otherwise be cut into many short chunks (2 blocks per wave) whose merge
  // outweighs the parallelism (B=1, ctx 16384: 64 chunks of 16 blocks 21.9 us, 32 of
  // 32 blocks 17.3 us).
  auto chunk_quads = [&](uint32_t nq, size_t cbk) {
    uint32_t cq = static_cast<uint32_t>(std::max<size_t>((cbk + 3) / 4, (nq + yx::kMaxChunks - 1) / yx::kMaxChunks));
    if (c->target_waves == 0) cq = std::max(cq, std::min<uint32_t>(yx::kBalQuads, (nq + kFanIn - 1) / kFanIn));
    if (tiny) cq = std::max<uint32_t>(cq, (nq + 7) / 8);
    return cq;
  };
  // Whether every chunk's blocks split evenly over kWideWaves waves.
  auto exact_split = [&](size_t cbk) {
    auto check = [&](uint32_t nblocks) {
      const uint32_t nq = (nblocks + 3) / 4, cq = chunk_quads(nq, cbk), nch = (nq + cq - 1) / cq;
      for (uint32_t ch = 0; ch < nch; ++ch) {
        const uint32_t b0 = 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * ch / nch);
        const uint32_t b1 = std::min(nblocks, 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * (ch + 1) / nch));
        if ((b1 - b0) % yx::kWideWaves != 0) return false;
      }
      return true;
    };
    for (const Sub& sb : subs)
      if (!check(sb.b1 - sb.b0)) return false;
    for (const Casc& cc : cascs)
      if (!check(cc.blocks)) return false;
    return true;
  };
  // Mid-size passes whose split is not exact anyway: work items of at least
  // kMinItemBlocks blocks (five per wave) while that still gives work to more than half
  // the CUs; shorter items spend more of their time in the start and the split-K
  // hand-off than they save in parallelism (B=12 ctx 2048, 6.1k blocks: 24-block items
  // 19.9 us, 40-block items 13.8; B=6 ctx 4096 20.5 -> 15.0; cfg2 22.0 -> 17.7; 48- and
  // 56-block minimums measured slower). Exact splits (the headline; B=8, ctx 4096) and
  // small passes keep one item per CU.
  constexpr size_t kMinItemBlocks = 40;
  if (c->target_waves == 0 && nt == 1 && work >= static_cast<size_t>(c->cus) * kMinItemBlocks / 2 &&
      !exact_split(cb))
    cb = std::max<size_t>(cb, kMinItemBlocks);
  // Each wave's page ids fit its 64 lanes: at most 64 blocks per wave.
  cb = std::max<size_t>(1, std::min<size_t>({cb, static_cast<size_t>(c->max_chunk_blocks), 64 * waves}));

  AttnPlan plan;
  plan.nt = static_cast<int>(nt);
  plan.wide = wide || !cascs.empty();
  size_t slot = 0;
  // The shared prefixes' items first (they are the longest-lived inputs of their
  // groups' merges); their partial slots always exist.
  std::vector<uint32_t> casc_base(cascs.size()), casc_nch(cascs.size()), casc_moff(cascs.size());
  for (size_t ci = 0; ci < cascs.size(); ++ci) {
    const Casc& cc = cascs[ci];
    const uint32_t nq = (cc.blocks + 3) / 4;
    const uint32_t cq = chunk_quads(nq, cb);
    if (cq * 4 > 64 * waves)  // each wave's page ids fit its 64 lanes
      return fail(YX_ERR_UNSUPPORTED, "shared prefix too long for 256 chunks of the widest work item");
    const uint32_t nch = (nq + cq - 1) / cq;
    casc_base[ci] = static_cast<uint32_t>(slot);
    casc_nch[ci] = nch;
    const uint32_t moff = static_cast<uint32_t>(plan.members.size());
    casc_moff[ci] = moff;
    for (uint32_t k = cc.first; k < cc.first + cc.count; ++k) {
      yx::SubRef m{};
      m.r0 = subs[k].r0;
      m.nrows = subs[k].n;
      m.counter = k;
      m.row_off = subs[k].r0 - cc.r0;
      plan.members.push_back(m);  // part_base and nch are set with the group's items
    }
    for (uint32_t ch = 0; ch < nch; ++ch) {
      yx::AttnItem w{};
      w.r0 = cc.r0;
      w.nrows = cc.n;
      w.pt_off = cc.dev_off;
      w.blk0 = 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * ch / nch);
      w.blk1 = std::min(cc.blocks, 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * (ch + 1) / nch));
      w.chunk = ch;
      w.nch = nch;
      w.part_base = static_cast<uint32_t>(slot);
      w.pref_base = moff;
      w.pref_nch = cc.count;
      w.pref_info = yx::kPrefixItem;
      plan.items.push_back(w);
    }
    slot += nch;
  }
  for (size_t si = 0; si < subs.size(); ++si) {
    const Sub& s = subs[si];
    // Chunks start on quads of blocks (the waves split them in quads), at most
    // kMaxChunks of them.
    const uint32_t nq = (s.b1 - s.b0 + 3) / 4;
    const uint32_t cq = chunk_quads(nq, cb);
    if (cq * 4 > 64 * waves)
      return fail(YX_ERR_UNSUPPORTED, "context too long for 256 chunks of the widest work item");
    const uint32_t nch = (nq + cq - 1) / cq;
    for (uint32_t ch = 0; ch < nch; ++ch) {
      yx::AttnItem w{};
      w.r0 = s.r0;
      w.nrows = s.n;
      w.pt_off = s.dev_off;
      w.blk0 = s.b0 + 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * ch / nch);
      w.blk1 = std::min(s.b1, s.b0 + 4 * static_cast<uint32_t>(static_cast<uint64_t>(nq) * (ch + 1) / nch));
      w.chunk = ch;
      w.nch = nch;
      w.part_base = static_cast<uint32_t>(slot);
      w.counter = static_cast<uint32_t>(si);
      if (s.casc >= 0) {
        w.pref_base = casc_base[s.casc];
        w.pref_nch = casc_nch[s.casc];
        w.pref_info = s.r0 - cascs[s.casc].r0;
      }
      plan.items.push_back(w);
    }
    if (s.casc >= 0) {  // the prefix items' view of this group's own chunks
      yx::SubRef& m = plan.members[casc_moff[s.casc] + (si - cascs[s.casc].first)];
      m.part_base = static_cast<uint32_t>(slot);
      m.nch = nch;
    }
    const uint32_t total = nch + (s.casc >= 0 ? casc_nch[s.casc] : 0);
    if (total > 1) slot += nch;
  }
  // XCD placement of shared prefixes: the GPU deals a launch's workgroups to its 8 XCDs
  // (each with its own L2) in turn, x fastest, so items x and x' of one KV head run on
  // one XCD when x = x' (mod 8). The prefix items reading the same chunk of a shared
  // prefix (chunk j of every prefix group of that prefix's run) take positions
  // = j (mod 8), so they share one L2 and the chunk comes from HBM once, not once per
  // XCD they landed on. The other items fill the remaining positions in their order.
  if (!cascs.empty() && c->xcd_prefix) {
    const size_t n = plan.items.size();
    std::vector<yx::AttnItem> placed(n);
    std::vector<char> taken(n, 0), moved(n, 0);
    size_t cursor[8] = {0, 1, 2, 3, 4, 5, 6, 7};
    bool ok = true;
    for (size_t i = 0; i < n && ok; ++i) {
      const yx::AttnItem& w = plan.items[i];
      if (!(w.pref_info & yx::kPrefixItem)) continue;
      const uint32_t r = w.chunk % 8;
      while (cursor[r] < n && taken[cursor[r]]) cursor[r] += 8;
      if (cursor[r] >= n) {
        ok = false;
        break;
      }
      placed[cursor[r]] = w;
      taken[cursor[r]] = 1;
      moved[i] = 1;
      cursor[r] += 8;
    }
    if (ok) {
      size_t pos = 0;
      for (size_t i = 0; i < n; ++i) {
        if (moved[i]) continue;
        while (taken[pos]) ++pos;
        placed[pos] = plan.items[i];
        taken[pos] = 1;
      }
      plan.items = std::move(placed);
    }
  }
  // The fused append needs each group in one sub and the last chunk of each group to
  // hold all of its rows' keys (the first row's position is the smallest).
  plan.fusable = true;
  {
    size_t gi = 0;
    for (const Sub& sb : subs) {
      while (c->groups[gi].r0 + c->groups[gi].n <= sb.r0) ++gi;
      if (sb.n != c->groups[gi].n) plan.fusable = false;
    }
    for (const yx::AttnItem& w : plan.items) {
      if (w.chunk + 1 != w.nch || (w.pref_info & yx::kPrefixItem)) continue;
      uint32_t pmin = UINT32_MAX;
      for (uint32_t i = w.r0; i < w.r0 + w.nrows; ++i) pmin = std::min(pmin, c->pos[i]);
      if (w.blk0 * 16 > pmin) plan.fusable = false;
    }
  }
  plan.f32 = f32;
  plan.balanced = !f32 && nt == 1 && c->decode_shape == 0;
  for (const yx::AttnItem& w : plan.items)
    if (w.blk1 - w.blk0 > 4 * yx::kBalQuads) plan.balanced = false;
  plan.small_units = plan.balanced;
  for (const yx::AttnItem& w : plan.items)
    if (w.blk1 - w.blk0 > 2 * yx::kBalQuads) plan.small_units = false;
  // One tile: the 16-row-tile kernel's static split of blocks over its waves where that
  // split is exact (every item's blocks a multiple of the waves) or the items are too
  // long for the queue; the queue kernel where waves would otherwise get unequal shares.
  // (Measured: B=16 ctx 4096, 64-block items, 25.9 against 26.3 us; cfg4's 128-block
  // items 47.3 against 48.4; cfg2's ~44-block items 25.4 against 24.9.)
  if (!f32 && nt == 1 && c->decode_shape == 0) {
    bool exact = true;
    for (const yx::AttnItem& w : plan.items)
      if ((w.blk1 - w.blk0) % yx::kWideWaves != 0) exact = false;
    plan.wide = !cascs.empty() || exact || !plan.balanced;
  }
  plan.slots = slot;
  plan.counters = subs.size();
  if (plan.items.size() > 0x7fffffff) return fail(YX_ERR_UNSUPPORTED, "too many work items");
  auto& p = c->plans[key];
  p = std::move(plan);
  p.cascades = cascs.size();
  *out = &p;
  return YX_OK;
}

// The device copy of a plan's work list (and shared-prefix member list), uploaded once
// per pass into buffers of the context (reused across passes).
int upload_plan(yx_ctx* c, AttnPlan* p) {
  if (p->uploaded) return YX_OK;
  const void* items = p->prefill ? static_cast<const void*>(p->pitems.data()) : p->items.data();
  const size_t ib = p->item_bytes();
  p->d_items = c->take_spare();
  int rc = p->d_items.ensure(std::max<size_t>(ib, 16), c->stream);
  if (rc) return rc;
  if ((rc = c->staging[c->cur_staging].upload(p->d_items.p, items, ib, c->stream))) return rc;
  p->dev_items = p->d_items.p;
  if (!p->members.empty()) {
    p->d_members = c->take_spare();
    if ((rc = p->d_members.ensure(p->members.size() * sizeof(yx::SubRef), c->stream))) return rc;
    rc = c->staging[c->cur_staging].upload(p->d_members.p, p->members.data(),
                                           p->members.size() * sizeof(yx::SubRef), c->stream);
    if (rc) return rc;
    p->dev_members = p->d_members.p;
  }
  p->uploaded = true;
  return YX_OK;
}

int append_impl(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v);

int qk_rope_impl(yx_ctx* c, yx_kv* kv, size_t layer, const yx::QkvIn& in, size_t hq, float* q_out,
                 bool kv_only = false);

// Attention of the pass's rows; with knew/vnew, the rows' K/V are stored first (in
// the same kernel when the plan allows it, else by the append kernel before it); with
// qkv, write_rows runs first (in the same kernel when the plan allows it, else as its
// own launch into a scratch q).
// noalloc: the work list, partials and counters live in the library's static scratch
// array instead of buffers of the context, so the call allocates no device or pinned
// memory (the entry point that allocates nothing).
int attention_impl(yx_ctx* c, yx_kv* kv, size_t layer, const float* q, float* out, size_t hq,
                   size_t hkv, size_t window, float scale, const float* knew = nullptr,
                   const float* vnew = nullptr, const yx::QkvIn* qkv = nullptr,
                   bool noalloc = false) {
  int rc = check_kv(c, kv, layer);
  if (rc) return rc;
  if (hkv != kv->hkv) return fail(YX_ERR_INVALID, "hkv differs from the arena's");
  if (hq == 0 || hq % hkv != 0) return fail(YX_ERR_INVALID, "hq must be a positive multiple of hkv");
  if (c->rows == 0) return YX_OK;
  if (!out || (!q && !qkv)) return fail(YX_ERR_INVALID, "null q or out");
  AttnPlan* plan;
  if (c->capturing && !c->plans.count(std::make_tuple(window, hq, hkv, kv->f32, kv->page)))
    return fail(YX_ERR_INVALID, "run the call once before capturing it (its work list is uploaded then)");
  if ((rc = build_plan(c, window, hq, hkv, kv->f32, kv->page, &plan))) return rc;
  {
    const auto key = std::make_tuple(window, hq, hkv, kv->f32, kv->page);
    if (std::find(c->used_keys.begin(), c->used_keys.end(), key) == c->used_keys.end())
      c->used_keys.push_back(key);
  }
  // Logical rows per partial slot: the kernel's tile rows.
  const size_t rps = plan->prefill ? static_cast<size_t>(!plan->f32 ? yx::kPrefillRows
                                                       : plan->pf32_waves == 4 ? yx::kPf32SmallRows
                                                                               : yx::kPf32Rows)
                    : plan->wide    ? static_cast<size_t>((plan->nt + 1) / 2) * 16
                                    : static_cast<size_t>(plan->nt) * 8;
  const size_t po_need = plan->slots * hkv * rps * 128 * 4, pml_need = plan->slots * hkv * rps * 8;
  const size_t cnt_need = plan->counters * hkv * 4 * yx::kCounterStride;
  const void* d_items;
  const yx::SubRef* d_members = nullptr;
  float* po;
  float2* pml;
  uint32_t* cnt;
  size_t po_cap, pml_cap;
  if (noalloc) {
    ScratchMap m;
    if ((rc = scratch_map(c, pml_need, po_need, cnt_need, &m))) return rc;
    if ((rc = scratch_take(c, std::make_tuple(window, hq, hkv, kv->f32, kv->page), plan, &m))) return rc;
    d_items = m.items;
    d_members = plan->members.empty() ? nullptr : static_cast<const yx::SubRef*>(m.members);
    po = static_cast<float*>(m.part_o);
    pml = static_cast<float2*>(m.part_ml);
    cnt = static_cast<uint32_t*>(m.counters);
    po_cap = std::max<size_t>(po_need, 16);
    pml_cap = std::max<size_t>(pml_need, 16);
  } else {
    if ((rc = upload_plan(c, plan))) return rc;
    if ((rc = c->part_o.ensure(std::max<size_t>(1, po_need), c->stream))) return rc;
    if ((rc = c->part_ml.ensure(std::max<size_t>(1, pml_need), c->stream))) return rc;
    if ((rc = c->counters.ensure(std::max<size_t>(1, cnt_need), c->stream, true))) return rc;
    d_items = plan->dev_items;
    d_members = plan->members.empty() ? nullptr : static_cast<const yx::SubRef*>(plan->dev_members);
    po = static_cast<float*>(c->part_o.p);
    pml = static_cast<float2*>(c->part_ml.p);
    cnt = static_cast<uint32_t*>(c->counters.p);
    po_cap = c->part_o.cap;
    pml_cap = c->part_ml.cap;
  }
  if (knew && (plan->prefill || !plan->fusable)) {
    if ((rc = append_impl(c, kv, layer, knew, vnew))) return rc;
    knew = vnew = nullptr;
  }
  if (qkv && plan->prefill && !plan->f32) {
    // The f16 prefill kernel normalises and rotates its rows' q heads itself; K/V first.
    if ((rc = qk_rope_impl(c, kv, layer, *qkv, hq, nullptr, true))) return rc;
  } else if (qkv && (plan->f32 || !(plan->fusable && (plan->wide ? plan->nt <= 2 : plan->balanced)))) {
    // (Two-tile passes keep write_rows as its own launch: fused, each work item
    // normalises and rotates up to 32 q heads before its first block, and cfg5's
    // Backend::attention took 28.9 us in one launch against 28.5 in two.)
    if ((rc = c->io_q.ensure(std::max<size_t>(16, c->rows * hq * 128 * 4), c->stream))) return rc;
    if ((rc = qk_rope_impl(c, kv, layer, *qkv, hq, static_cast<float*>(c->io_q.p)))) return rc;
    q = static_cast<const float*>(c->io_q.p);
    qkv = nullptr;
  }
  if (plan->prefill) {
    uint32_t shift = 0;
    while ((16u << shift) < kv->page) ++shift;
    hipEvent_t e0;
    if ((rc = prof_begin(c, YX_KERNEL_ATTENTION, &e0))) return rc;
    const dim3 pgrid(static_cast<unsigned>(plan->pitems.size() * hkv));
    if (po_cap > 0xffffffffu || pml_cap > 0xffffffffu)
      return fail(YX_ERR_UNSUPPORTED, "prefill partials beyond 4 GiB");
    const uint32_t pf_po_bytes = static_cast<uint32_t>(po_cap), pf_pml_bytes = static_cast<uint32_t>(pml_cap);
    if (plan->f32) {
      auto* kern = plan->pf32_waves == 4 ? yx::paged_attn_prefill_f32<4> : yx::paged_attn_prefill_f32<8>;
      hipLaunchKernelGGL(kern, pgrid, dim3(64 * plan->pf32_waves), 0, c->stream,
                         static_cast<const yx::PrefillItem*>(d_items), c->dev_pos,
                         static_cast<const uint32_t*>(c->d_pages.p),
                         reinterpret_cast<const float*>(kv->k[layer]),
                         reinterpret_cast<const float*>(kv->v[layer]), q, out,
                         static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv), shift,
                         static_cast<uint32_t>(window), scale * yx::kLog2e, po, pml, cnt,
                         pf_po_bytes, pf_pml_bytes);
    } else if (qkv)
      hipLaunchKernelGGL((yx::paged_attn_prefill<true>), pgrid, dim3(64 * yx::kPrefillWaves), 0, c->stream,
                       static_cast<const yx::PrefillItem*>(d_items),
                       c->dev_pos, static_cast<const uint32_t*>(c->d_pages.p),
                       kv->k[layer], kv->v[layer], q, out, static_cast<uint32_t>(hq),
                       static_cast<uint32_t>(hkv), shift, static_cast<uint32_t>(window),
                       scale * yx::kLog2e, *qkv, po, pml, cnt, pf_po_bytes, pf_pml_bytes);
    else
      hipLaunchKernelGGL((yx::paged_attn_prefill<false>), pgrid, dim3(64 * yx::kPrefillWaves), 0, c->stream,
                       static_cast<const yx::PrefillItem*>(d_items),
                       c->dev_pos, static_cast<const uint32_t*>(c->d_pages.p),
                       kv->k[layer], kv->v[layer], q, out, static_cast<uint32_t>(hq),
                       static_cast<uint32_t>(hkv), shift, static_cast<uint32_t>(window),
                       scale * yx::kLog2e, yx::QkvIn{}, po, pml, cnt, pf_po_bytes, pf_pml_bytes);
    YX_HIP(hipGetLastError());
    return prof_end(c, YX_KERNEL_ATTENTION, e0);
  }
  // write_rows runs in the same launch in the queue kernel and the one-tile wide kernel
  // only (qkv was cleared above otherwise).
  if (qkv && (plan->f32 || !(plan->wide ? plan->nt <= 2 : plan->balanced)))
    return fail(YX_ERR_INVALID, "internal: write_rows cannot be fused here");
  const float scale_log2 = scale * yx::kLog2e;
  dim3 grid(static_cast<unsigned>(plan->items.size()), static_cast<unsigned>(hkv));
  hipEvent_t e0;
  if ((rc = prof_begin(c, YX_KERNEL_ATTENTION, &e0))) return rc;
  const auto* items = static_cast<const yx::AttnItem*>(d_items);
  const auto* pos = c->dev_pos;
  const auto* pages = static_cast<const uint32_t*>(c->d_pages.p);
  const uint32_t H = static_cast<uint32_t>(hq), HK = static_cast<uint32_t>(hkv);
  uint32_t P = 0;
  while ((16u << P) < kv->page) ++P;  // log2(blocks of 16 keys per page)
  const uint32_t W = static_cast<uint32_t>(window);
  const uint32_t po_bytes = static_cast<uint32_t>(std::min<size_t>(po_cap, 0xffffffffu));
  const uint32_t pml_bytes = static_cast<uint32_t>(std::min<size_t>(pml_cap, 0xffffffffu));
  const auto* mem = d_members;
#define YX_LAUNCH_DECODE(NT)                                                                        \
  hipLaunchKernelGGL(yx::paged_attn_decode<NT>, grid, dim3(64 * yx::DecodeWaves<NT>::value), 0,      \
                     c->stream, items, pos, pages,                                                  \
                     kv->k[layer], kv->v[layer], q, out, po, pml, cnt, knew, vnew,                 \
                     c->dev_slot, kv->k[layer], kv->v[layer],       \
                     po_bytes, pml_bytes, H, HK, P, W, scale_log2)
  if (plan->f32) {
    hipLaunchKernelGGL(yx::paged_attn_decode_f32, grid, dim3(64 * yx::kWideWaves), 0, c->stream,
                       items, pos, pages, kv->kf(layer), kv->vf(layer), q, out, po, pml, cnt, knew,
                       vnew, c->dev_slot, kv->kf(layer),
                       kv->vf(layer), po_bytes, pml_bytes, H, HK, P, W, scale_log2, mem);
  } else if (plan->balanced && !plan->wide) {
#define YX_LAUNCH_BAL(QKV, UB, KN, VN, IN)                                                          \
  hipLaunchKernelGGL((yx::paged_attn_decode_balanced<QKV, UB>), grid, dim3(64 * yx::kBalWaves), 0,  \
                     c->stream, items, pos, pages, kv->k[layer], kv->v[layer], q, out, po, pml,     \
                     cnt, KN, VN, c->dev_slot, kv->k[layer],        \
                     kv->v[layer], po_bytes, pml_bytes, H, HK, P, W, scale_log2, IN)
    if (qkv && plan->small_units) YX_LAUNCH_BAL(true, 2, nullptr, nullptr, *qkv);
    else if (qkv) YX_LAUNCH_BAL(true, 4, nullptr, nullptr, *qkv);
    else if (plan->small_units) YX_LAUNCH_BAL(false, 2, knew, vnew, yx::QkvIn{});
    else YX_LAUNCH_BAL(false, 4, knew, vnew, yx::QkvIn{});
#undef YX_LAUNCH_BAL
  } else if (plan->wide) {
#define YX_LAUNCH_WIDE(NT, QKV, KN, VN, IN, CASC)                                                   \
  hipLaunchKernelGGL((yx::paged_attn_decode_wide<NT, QKV, CASC>), grid, dim3(64 * yx::kWideWaves), 0, \
                     c->stream, items, pos, pages, kv->k[layer], kv->v[layer], q, out, po, pml,     \
                     cnt, KN, VN, c->dev_slot, kv->k[layer],        \
                     kv->v[layer], po_bytes, pml_bytes, H, HK, P, W, scale_log2, IN, mem)
    const bool casc = plan->cascades > 0;  // shared prefixes only in one-tile passes
    if (qkv && casc) YX_LAUNCH_WIDE(1, true, nullptr, nullptr, *qkv, true);
    else if (qkv) YX_LAUNCH_WIDE(1, true, nullptr, nullptr, *qkv, false);
    else if (plan->nt <= 2 && casc) YX_LAUNCH_WIDE(1, false, knew, vnew, yx::QkvIn{}, true);
    else if (plan->nt <= 2) YX_LAUNCH_WIDE(1, false, knew, vnew, yx::QkvIn{}, false);
    else YX_LAUNCH_WIDE(2, false, knew, vnew, yx::QkvIn{}, false);
#undef YX_LAUNCH_WIDE
  } else switch (plan->nt) {
    case 1: YX_LAUNCH_DECODE(1); break;
    case 2: YX_LAUNCH_DECODE(2); break;
    default: YX_LAUNCH_DECODE(3); break;
  }
#undef YX_LAUNCH_DECODE
  YX_HIP(hipGetLastError());
  return prof_end(c, YX_KERNEL_ATTENTION, e0);
}

int append_impl(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v) {
  int rc = check_kv(c, kv, layer);
  if (rc) return rc;
  if (c->rows == 0) return YX_OK;
  if (!k || !v) return fail(YX_ERR_INVALID, "null k or v");
  const size_t threads = c->rows * kv->hkv * 16;
  dim3 grid(static_cast<unsigned>((threads + 255) / 256), 2);
  hipEvent_t e0;
  if ((rc = prof_begin(c, YX_KERNEL_APPEND, &e0))) return rc;
  if (kv->f32) {
    dim3 grid32(static_cast<unsigned>((threads * 2 + 255) / 256), 2);
    hipLaunchKernelGGL(yx::kv_append_f32, grid32, dim3(256), 0, c->stream, k, v,
                       c->dev_slot, kv->kf(layer), kv->vf(layer),
                       static_cast<uint32_t>(c->rows), static_cast<uint32_t>(kv->hkv),
                       static_cast<uint32_t>(kv->page));
  } else {
    hipLaunchKernelGGL(yx::kv_append_f16, grid, dim3(256), 0, c->stream, k, v,
                       c->dev_slot, kv->k[layer], kv->v[layer],
                       static_cast<uint32_t>(c->rows), static_cast<uint32_t>(kv->hkv),
                       static_cast<uint32_t>(kv->page));
  }
  YX_HIP(hipGetLastError());
  return prof_end(c, YX_KERNEL_APPEND, e0);
}

// Rows of the pass that write_rows can run on: positions inside the RoPE table (the
// page-table coverage is checked with the arena, check_kv).
int check_qkv_rows(yx_ctx* c, size_t rope_len) {
  if (rope_len > 0xffffffffu) return fail(YX_ERR_UNSUPPORTED, "RoPE table too long");
  for (size_t i = 0; i < c->rows; ++i)
    if (c->pos[i] >= rope_len) return fail(YX_ERR_INVALID, "a row's position is beyond the RoPE table");
  return YX_OK;
}

// write_rows on its own: workgroups of kRopeVecs head vectors; with kv_only, the key
// and value heads only (q_out unused).
int qk_rope_impl(yx_ctx* c, yx_kv* kv, size_t layer, const yx::QkvIn& in, size_t hq, float* q_out,
                 bool kv_only) {
  if (c->rows == 0) return YX_OK;
  const size_t hkv = kv->hkv;
  const size_t nvec = c->rows * (kv_only ? hkv : hq + hkv);
  if (nvec > 0xffffffffu) return fail(YX_ERR_UNSUPPORTED, "too many head vectors in the pass");
  dim3 grid(static_cast<unsigned>((nvec + yx::kRopeVecs - 1) / yx::kRopeVecs));
  uint32_t page_shift = 0;
  while ((1u << page_shift) < kv->page) ++page_shift;
  hipEvent_t e0;
  int rc;
  if ((rc = prof_begin(c, YX_KERNEL_QK_ROPE, &e0))) return rc;
  if (kv->f32)
    hipLaunchKernelGGL(yx::qk_norm_rope_append<float>, grid, dim3(yx::kRopeThreads), 0, c->stream,
                       in.qkv, in.q_norm, in.k_norm, in.rope_cs, in.rope_len, in.eps,
                       c->dev_pos, c->dev_slot,
                       kv->kf(layer), kv->vf(layer), q_out, static_cast<uint32_t>(hq),
                       static_cast<uint32_t>(hkv), page_shift, static_cast<uint32_t>(nvec),
                       static_cast<uint32_t>(kv_only ? hq : 0));
  else
    hipLaunchKernelGGL(yx::qk_norm_rope_append<_Float16>, grid, dim3(yx::kRopeThreads), 0, c->stream,
                       in.qkv, in.q_norm, in.k_norm, in.rope_cs, in.rope_len, in.eps,
                       c->dev_pos, c->dev_slot,
                       kv->k[layer], kv->v[layer], q_out, static_cast<uint32_t>(hq),
                       static_cast<uint32_t>(hkv), page_shift, static_cast<uint32_t>(nvec),
                       static_cast<uint32_t>(kv_only ? hq : 0));
  YX_HIP(hipGetLastError());
  return prof_end(c, YX_KERNEL_QK_ROPE, e0);
}

}  // namespace

extern "C" {

const char* yx_last_error(void) { return g_err.c_str(); }

#ifdef YX_PF_PROF
// Profiling build only: reads and clears the prefill kernel's phase clocks.
int yx_debug_pf_prof(unsigned long long* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(yx::g_pf_prof), sizeof(yx::g_pf_prof)) == hipSuccess ? 0 : 5;
}
#endif

int yx_device_count(int* n) {
  YX_HIP(hipGetDeviceCount(n));
  return YX_OK;
}

int yx_ctx_create(int device, yx_ctx** out) {
  if (!out) return fail(YX_ERR_INVALID, "null output");
  int n = 0;
  YX_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(YX_ERR_INVALID, "no such device");
  hipDeviceProp_t prop;
  YX_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(YX_ERR_UNSUPPORTED, std::string("the kernels are built for gfx950, not ") + prop.gcnArchName);
  auto* c = new yx_ctx();
  c->device = device;
  c->cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&c->t0);
  if (e == hipSuccess) e = hipEventCreate(&c->t1);
  if (e != hipSuccess) {
    delete c;
    return fail(YX_ERR_HIP, std::string("context set-up: ") + hipGetErrorString(e));
  }
  if (int rc = scratch_init(device, c->stream)) {
    yx_ctx_destroy(c);
    return rc;
  }
  *out = c;
  return YX_OK;
}

int yx_ctx_destroy(yx_ctx* c) {
  if (!c) return YX_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  scratch_forget(c, c->device);
  for (auto& p : c->prof)
    for (auto& e : p.pending) {
      (void)hipEventDestroy(e.first);
      (void)hipEventDestroy(e.second);
    }
  for (auto& kv : c->plans) {
    kv.second.d_items.release();
    kv.second.d_members.release();
  }
  for (DevBuf& b : c->spare) b.release();
  c->spare.clear();
  for (DevBuf* b : {&c->d_meta, &c->d_pages, &c->am_keys, &c->am_counters, &c->mm_part, &c->mm_counters,
                    &c->part_o, &c->part_ml, &c->counters,
                    &c->io_a, &c->io_b, &c->io_c, &c->io_q})
    b->release();
  if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
  if (c->graph) (void)hipGraphDestroy(c->graph);
  c->staging[0].release();
  c->staging[1].release();
  (void)hipEventDestroy(c->t0);
  (void)hipEventDestroy(c->t1);
  (void)hipStreamDestroy(c->stream);
  delete c;
  return YX_OK;
}

int yx_sync(yx_ctx* c) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_ctx_set_option(yx_ctx* c, const char* key, long value) {
  if (!c || !key) return fail(YX_ERR_INVALID, "null argument");
  if (value < 0 || (value == 0 && std::strcmp(key, "attn_target_waves") &&
                    std::strcmp(key, "attn_decode_shape") && std::strcmp(key, "attn_cascade") &&
                    std::strcmp(key, "attn_xcd_prefix") &&
                    std::strcmp(key, "prefill_split") && std::strcmp(key, "prefill_min_rows") &&
                    std::strcmp(key, "matmul_k_split") && std::strcmp(key, "argmax_slices") &&
                    std::strcmp(key, "prefill_f32_waves")))
    return fail(YX_ERR_INVALID,
                "option values are positive (attn_target_waves, attn_decode_shape, prefill_min_rows, "
                "matmul_k_split, argmax_slices: 0 = automatic; attn_cascade, prefill_split: 0 = off)");
  if (!std::strcmp(key, "attn_target_waves"))
    c->target_waves = value;
  else if (!std::strcmp(key, "attn_max_tiles"))
    c->max_tiles = std::min<long>(value, 4);
  else if (!std::strcmp(key, "attn_decode_shape"))
    c->decode_shape = std::min<long>(value, 2);
  else if (!std::strcmp(key, "prefill_min_rows"))
    c->prefill_min_rows = value;
  else if (!std::strcmp(key, "attn_max_chunk_blocks"))
    c->max_chunk_blocks = value;
  else if (!std::strcmp(key, "attn_xcd_prefix"))
    c->xcd_prefix = value;
  else if (!std::strcmp(key, "attn_cascade"))
    c->cascade = value ? 1 : 0;
  else if (!std::strcmp(key, "prefill_split"))
    c->prefill_split = value ? 1 : 0;
  else if (!std::strcmp(key, "matmul_k_split"))
    c->matmul_k_split = std::min<long>(value, 64);
  else if (!std::strcmp(key, "prefill_f32_waves")) {
    if (value != 0 && value != 4 && value != 8) return fail(YX_ERR_INVALID, "prefill_f32_waves is 0, 4 or 8");
    c->pf32_waves = value;
  } else if (!std::strcmp(key, "argmax_slices"))
    c->argmax_slices = std::min<long>(value, 1024);
  else
    return fail(YX_ERR_INVALID, std::string("unknown option ") + key);
  ++c->epoch;
  c->retire_plans();
  return YX_OK;
}

int yx_kv_create(yx_ctx* c, size_t layers, size_t pages, size_t page_size, size_t hkv,
                 size_t head_dim, int dtype, yx_kv** out) {
  if (!c || !out) return fail(YX_ERR_INVALID, "null argument");
  if (dtype != YX_DTYPE_F16 && dtype != YX_DTYPE_F32) return fail(YX_ERR_UNSUPPORTED, "dtype must be f16 or f32");
  if (head_dim != 128) return fail(YX_ERR_UNSUPPORTED, "head_dim must be 128");
  if (page_size < 16 || (page_size & (page_size - 1)) != 0)
    return fail(YX_ERR_UNSUPPORTED, "page size must be a power of two, at least 16");
  if (layers == 0 || pages == 0 || hkv == 0) return fail(YX_ERR_INVALID, "empty arena");
  if (pages > 0xffffffffull / page_size) return fail(YX_ERR_INVALID, "arena slots are 32-bit");
  int rc = c->set_device();
  if (rc) return rc;
  auto* kv = new yx_kv();
  kv->layers = layers;
  kv->pages = pages;
  kv->page = page_size;
  kv->hkv = hkv;
  kv->d = head_dim;
  kv->f32 = dtype == YX_DTYPE_F32;
  const size_t bytes = pages * kv->page_bytes();
  std::vector<void*> bases;
  for (size_t l = 0; l < layers; ++l) {
    void *kp = nullptr, *vp = nullptr;
    hipError_t e = hipMalloc(&kp, bytes);
    if (e == hipSuccess) e = hipMalloc(&vp, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(kp, 0, bytes, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(vp, 0, bytes, c->stream);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // as in YX_HIP
      if (kp) (void)hipFree(kp);
      if (vp) (void)hipFree(vp);
      yx_kv_destroy(c, kv);
      return fail(YX_ERR_HIP, std::string("KV arena allocation: ") + hipGetErrorString(e));
    }
    kv->k.push_back(static_cast<_Float16*>(kp));
    kv->v.push_back(static_cast<_Float16*>(vp));
    bases.push_back(kp);
    bases.push_back(vp);
  }
  if ((rc = kv->bases.ensure(bases.size() * sizeof(void*), c->stream))) {
    yx_kv_destroy(c, kv);
    return rc;
  }
  YX_HIP(hipMemcpyAsync(kv->bases.p, bases.data(), bases.size() * sizeof(void*),
                        hipMemcpyHostToDevice, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  *out = kv;
  return YX_OK;
}

int yx_kv_destroy(yx_ctx* c, yx_kv* kv) {
  if (!kv) return YX_OK;
  if (c) {
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    ++c->epoch;
  }
  for (auto* p : kv->k) (void)hipFree(p);
  for (auto* p : kv->v) (void)hipFree(p);
  kv->bases.release();
  delete kv;
  return YX_OK;
}

int yx_kv_layer_ptr(yx_kv* kv, size_t layer, int which, void** out) {
  if (!kv || !out || layer >= kv->layers) return fail(YX_ERR_INVALID, "bad arena, layer or output");
  *out = which == YX_K ? static_cast<void*>(kv->k[layer]) : static_cast<void*>(kv->v[layer]);
  return YX_OK;
}

size_t yx_kv_page_bytes(const yx_kv* kv) { return kv ? kv->page_bytes() : 0; }

int yx_kv_copy_pages(yx_ctx* c, yx_kv* kv, const uint32_t* src, const uint32_t* dst, size_t n) {
  if (!c || !kv) return fail(YX_ERR_INVALID, "null argument");
  if (n == 0) return YX_OK;
  if (!src || !dst) return fail(YX_ERR_INVALID, "null page list");
  for (size_t i = 0; i < n; ++i)
    if (src[i] >= kv->pages || dst[i] >= kv->pages) return fail(YX_ERR_INVALID, "page beyond the arena");
  int rc = c->set_device();
  if (rc) return rc;
  const uint32_t vec16 = static_cast<uint32_t>(kv->page_bytes() / 16);
  // Copies run in list order: a batch ends where a copy reads or writes a page an
  // earlier copy of the batch writes, or writes a page it reads.
  size_t i = 0;
  while (i < n) {
    CopyList list;
    std::vector<uint32_t> reads, writes;
    int m = 0;
    while (i < n && m < kMaxCopiesPerLaunch) {
      auto has = [](const std::vector<uint32_t>& s, uint32_t x) {
        return std::find(s.begin(), s.end(), x) != s.end();
      };
      if (has(writes, src[i]) || has(writes, dst[i]) || has(reads, dst[i])) break;
      list.src[m] = src[i];
      list.dst[m] = dst[i];
      reads.push_back(src[i]);
      writes.push_back(dst[i]);
      ++m;
      ++i;
    }
    hipEvent_t e0;
    if ((rc = prof_begin(c, YX_KERNEL_COPY, &e0))) return rc;
    hipLaunchKernelGGL(kv_copy_pages_list, dim3(m, static_cast<unsigned>(2 * kv->layers)), dim3(256), 0,
                       c->stream, list, static_cast<uint4* const*>(kv->bases.p), vec16);
    YX_HIP(hipGetLastError());
    if ((rc = prof_end(c, YX_KERNEL_COPY, e0))) return rc;
  }
  return YX_OK;
}

// Page contents through the host in the logical layout [hkv][page_size][128]; K is
// converted from / to the arena's block order (k_offset).
static int page_io(yx_ctx* c, yx_kv* kv, size_t layer, const uint32_t* pages, size_t n, void* k,
                   void* v, bool read) {
  if (!c || !kv || layer >= kv->layers) return fail(YX_ERR_INVALID, "bad arena or layer");
  if (n && !pages) return fail(YX_ERR_INVALID, "null page list");
  int rc = c->set_device();
  if (rc) return rc;
  const size_t pb = kv->page_bytes();
  const size_t ph = pb / 2;  // halves per page
  std::vector<uint16_t> tmp(ph);
  auto permute = [&](const uint16_t* logical, uint16_t* arena, bool to_arena) {
    for (size_t h = 0; h < kv->hkv; ++h)
      for (uint32_t off = 0; off < kv->page; ++off)
        for (uint32_t ch = 0; ch < 16; ++ch) {
          const size_t region = h * kv->page * 128;
          const uint16_t* src;
          uint16_t* dst;
          if (to_arena) {
            src = logical + region + off * 128 + ch * 8;
            dst = arena + region + yx::k_offset(off, ch);
          } else {
            src = arena + region + yx::k_offset(off, ch);
            dst = const_cast<uint16_t*>(logical) + region + off * 128 + ch * 8;
          }
          std::memcpy(dst, src, 16);
        }
  };
  for (size_t i = 0; i < n; ++i) {
    if (pages[i] >= kv->pages) return fail(YX_ERR_INVALID, "page beyond the arena");
    char* kd = reinterpret_cast<char*>(kv->k[layer]) + pages[i] * pb;
    char* vd = reinterpret_cast<char*>(kv->v[layer]) + pages[i] * pb;
    if (kv->f32) {  // K in V's layout: plain copies
      if (read) {
        if (k) YX_HIP(hipMemcpyAsync(static_cast<char*>(k) + i * pb, kd, pb, hipMemcpyDeviceToHost, c->stream));
        if (v) YX_HIP(hipMemcpyAsync(static_cast<char*>(v) + i * pb, vd, pb, hipMemcpyDeviceToHost, c->stream));
      } else {
        if (k) YX_HIP(hipMemcpyAsync(kd, static_cast<const char*>(k) + i * pb, pb, hipMemcpyHostToDevice, c->stream));
        if (v) YX_HIP(hipMemcpyAsync(vd, static_cast<const char*>(v) + i * pb, pb, hipMemcpyHostToDevice, c->stream));
      }
    } else if (read) {
      if (k) {
        YX_HIP(hipMemcpyAsync(tmp.data(), kd, pb, hipMemcpyDeviceToHost, c->stream));
        YX_HIP(hipStreamSynchronize(c->stream));
        permute(reinterpret_cast<uint16_t*>(static_cast<char*>(k) + i * pb), tmp.data(), false);
      }
      if (v) YX_HIP(hipMemcpyAsync(static_cast<char*>(v) + i * pb, vd, pb, hipMemcpyDeviceToHost, c->stream));
    } else {
      if (k) {
        permute(reinterpret_cast<const uint16_t*>(static_cast<const char*>(k) + i * pb), tmp.data(), true);
        YX_HIP(hipMemcpyAsync(kd, tmp.data(), pb, hipMemcpyHostToDevice, c->stream));
        YX_HIP(hipStreamSynchronize(c->stream));
      }
      if (v) YX_HIP(hipMemcpyAsync(vd, static_cast<const char*>(v) + i * pb, pb, hipMemcpyHostToDevice, c->stream));
    }
  }
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_kv_read_pages(yx_ctx* c, yx_kv* kv, size_t layer, const uint32_t* pages, size_t n,
                     void* k_out, void* v_out) {
  return page_io(c, kv, layer, pages, n, k_out, v_out, true);
}

int yx_kv_write_pages(yx_ctx* c, yx_kv* kv, size_t layer, const uint32_t* pages, size_t n,
                      const void* k_in, const void* v_in) {
  return page_io(c, kv, layer, pages, n, const_cast<void*>(k_in), const_cast<void*>(v_in), false);
}

int yx_pass_begin(yx_ctx* c, size_t rows, const uint32_t* pos, const uint32_t* kv_slot,
                  const uint32_t* pt_off, const uint32_t* pages, size_t npages) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  if (rows && (!pos || !kv_slot || !pt_off)) return fail(YX_ERR_INVALID, "null row metadata");
  if (npages && !pages) return fail(YX_ERR_INVALID, "null page tables");
  if (rows > 0x7fffffff || npages > 0x7fffffff) return fail(YX_ERR_INVALID, "pass too large");
  // Every key a row can see must have a page-table entry; a sequence's rows (one page
  // table) are consecutive.
  {
    std::unordered_set<uint32_t> seen;
    for (size_t i = 0; i < rows; ++i) {
      if (static_cast<uint64_t>(pt_off[i]) >= npages)
        return fail(YX_ERR_INVALID, "row page table offset beyond the page tables");
      if ((i == 0 || pt_off[i] != pt_off[i - 1]) && !seen.insert(pt_off[i]).second)
        return fail(YX_ERR_INVALID, "rows of one sequence are not consecutive");
    }
  }
  int rc = c->set_device();
  if (rc) return rc;
  c->have_pass = false;
  ++c->epoch;
  c->retire_plans();
  c->rows = rows;
  c->npages = npages;
  c->pos.assign(pos, pos + rows);
  c->slot.assign(kv_slot, kv_slot + rows);
  c->pt_off.assign(pt_off, pt_off + rows);
  c->pages.assign(pages, pages + npages);
  c->max_page = 0;
  for (uint32_t p : c->pages) c->max_page = std::max(c->max_page, p);
  c->max_slot = 0;
  for (uint32_t s : c->slot) c->max_slot = std::max(c->max_slot, s);
  c->groups.clear();
  for (size_t i = 0; i < rows; ++i) {
    if (!c->groups.empty() && c->groups.back().pt_off == pt_off[i])
      c->groups.back().n += 1;
    else
      c->groups.push_back(Group{static_cast<uint32_t>(i), 1, pt_off[i], 0});
  }
  c->cur_staging ^= 1;
  Staging& st = c->staging[c->cur_staging];
  if ((rc = st.reset())) return rc;

  // Page tables on the device: one region per group, entries [0, need) of the group's
  // table. A table runs to the next group's offset (or the end of the pass's tables) and
  // at least as far as the group's positions reach with the smallest page size, since a
  // table is followed by later ones (PassMeta::page_table). The previous pass's regions
  // are kept when there are as many groups and each fits its region; the regions are
  // then updated in place, entry runs that differ from what the device holds.
  const size_t ng = c->groups.size();
  std::vector<uint32_t> starts(pt_off, pt_off + rows);
  std::sort(starts.begin(), starts.end());
  starts.erase(std::unique(starts.begin(), starts.end()), starts.end());
  std::vector<uint32_t> need(ng);
  bool keep = c->region_off.size() == ng;
  for (size_t g = 0; g < ng; ++g) {
    const Group& gr = c->groups[g];
    auto nx = std::upper_bound(starts.begin(), starts.end(), gr.pt_off);
    const uint32_t len = (nx == starts.end() ? static_cast<uint32_t>(npages) : *nx) - gr.pt_off;
    uint32_t reach = 0;
    for (uint32_t r = gr.r0; r < gr.r0 + gr.n; ++r) reach = std::max(reach, pos[r] / 16 + 1);
    need[g] = std::min(static_cast<uint32_t>(npages) - gr.pt_off, std::max(len, reach));
    if (keep && need[g] > c->region_cap[g]) keep = false;
  }
  if (!keep) {
    size_t total = 0;
    c->region_off.assign(ng, 0);
    c->region_cap.assign(ng, 0);
    for (size_t g = 0; g < ng; ++g) {
      const size_t cap = (need[g] + std::max<size_t>(64, need[g] / 8) + 63) / 64 * 64;
      if (total + cap > 0x7fffffff) return fail(YX_ERR_INVALID, "pass too large");
      c->region_off[g] = static_cast<uint32_t>(total);
      c->region_cap[g] = static_cast<uint32_t>(cap);
      total += cap;
    }
    if ((rc = c->d_pages.ensure(std::max<size_t>(4, total * 4), c->stream))) return rc;
    c->dev_mirror.assign(total, 0xffffffffu);  // matches no page id: every entry is sent
  }
  std::vector<uint32_t> runs, data;  // runs of (device index, count, data index)
  for (size_t g = 0; g < ng; ++g) {
    c->groups[g].dev_off = c->region_off[g];
    const uint32_t* src = pages + c->groups[g].pt_off;
    uint32_t* mir = c->dev_mirror.data() + c->region_off[g];
    for (uint32_t j = 0; j < need[g]; ++j) {
      if (mir[j] == src[j]) continue;
      const uint32_t d = c->region_off[g] + j;
      if (!runs.empty() && runs[runs.size() - 3] + runs[runs.size() - 2] == d)
        ++runs[runs.size() - 2];
      else
        runs.insert(runs.end(), {d, 1u, static_cast<uint32_t>(data.size())});
      data.push_back(src[j]);
      mir[j] = src[j];
    }
  }
  const uint32_t nruns = static_cast<uint32_t>(runs.size() / 3);
  c->pages_sent += data.size();
  c->runs_sent += nruns;

  // The work lists of the attention calls the previous pass made are built now and go
  // in the same copy (a decode loop calls the same layers every step); other calls
  // build theirs at their first use.
  std::vector<AttnPlan*> pre;
  {
    auto keys = std::move(c->used_keys);
    c->used_keys.clear();
    for (const auto& k : keys) {
      AttnPlan* p = nullptr;
      if (build_plan(c, std::get<0>(k), std::get<1>(k), std::get<2>(k), std::get<3>(k), std::get<4>(k), &p) == YX_OK)
        pre.push_back(p);
    }
  }

  // One copy: positions, slots, page-table runs and data, prebuilt work lists.
  auto r256 = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t o = off;
    off += r256(b);
    return o;
  };
  const size_t o_pos = take(rows * 4), o_slot = take(rows * 4), o_runs = take(runs.size() * 4),
               o_data = take(data.size() * 4);
  std::vector<std::pair<size_t, size_t>> o_plan;
  for (AttnPlan* p : pre) {
    const size_t oi = take(p->item_bytes());
    o_plan.emplace_back(oi, take(p->members.size() * sizeof(yx::SubRef)));
  }
  const size_t total = std::max<size_t>(off, 256);
  if ((rc = c->d_meta.ensure(total, c->stream))) return rc;
  char* h = nullptr;
  if ((rc = st.reserve(total, &h))) return rc;
  std::memcpy(h + o_pos, pos, rows * 4);
  std::memcpy(h + o_slot, kv_slot, rows * 4);
  if (!runs.empty()) std::memcpy(h + o_runs, runs.data(), runs.size() * 4);
  if (!data.empty()) std::memcpy(h + o_data, data.data(), data.size() * 4);
  char* dm = static_cast<char*>(c->d_meta.p);
  for (size_t i = 0; i < pre.size(); ++i) {
    AttnPlan* p = pre[i];
    const void* items = p->prefill ? static_cast<const void*>(p->pitems.data()) : p->items.data();
    if (p->item_bytes()) std::memcpy(h + o_plan[i].first, items, p->item_bytes());
    if (!p->members.empty())
      std::memcpy(h + o_plan[i].second, p->members.data(), p->members.size() * sizeof(yx::SubRef));
    p->dev_items = dm + o_plan[i].first;
    p->dev_members = dm + o_plan[i].second;
    p->uploaded = true;
  }
  if ((rc = st.send(c->d_meta.p, off, c->stream))) return rc;
  c->dev_pos = reinterpret_cast<const uint32_t*>(dm + o_pos);
  c->dev_slot = reinterpret_cast<const uint32_t*>(dm + o_slot);
  if (nruns) {
    hipLaunchKernelGGL(page_runs_apply, dim3(std::min<uint32_t>(nruns, 256)), dim3(256), 0, c->stream,
                       reinterpret_cast<const uint32_t*>(dm + o_runs), nruns,
                       reinterpret_cast<const uint32_t*>(dm + o_data), static_cast<uint32_t*>(c->d_pages.p));
    YX_HIP(hipGetLastError());
  }
  c->have_pass = true;
  return YX_OK;
}

int yx_ctx_get_stat(yx_ctx* c, const char* key, uint64_t* out) {
  if (!c || !key || !out) return fail(YX_ERR_INVALID, "null argument");
  if (!std::strcmp(key, "page_entries_sent"))
    *out = c->pages_sent;
  else if (!std::strcmp(key, "page_runs_sent"))
    *out = c->runs_sent;
  else if (!std::strcmp(key, "prefill_split_tiles"))
    *out = c->split_tiles;
  else if (!std::strcmp(key, "prefill_plans"))
    *out = c->prefill_plans;
  else
    return fail(YX_ERR_INVALID, std::string("unknown statistic ") + key);
  return YX_OK;
}

int yx_kv_append_dev(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  return append_impl(c, kv, layer, k, v);
}

int yx_qk_rope_append_dev(yx_ctx* c, yx_kv* kv, size_t layer, const float* qkv,
                          const float* q_norm, const float* k_norm, const float* rope_cs,
                          size_t rope_len, float eps, size_t hq, size_t hkv, float* q_out) {
  if (!c || !kv || !qkv || !q_norm || !k_norm || !rope_cs || !q_out)
    return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  if ((rc = check_kv(c, kv, layer))) return rc;
  if (hkv != kv->hkv) return fail(YX_ERR_INVALID, "hkv differs from the arena's");
  if (hq == 0 || hq % hkv != 0) return fail(YX_ERR_INVALID, "hq must be a positive multiple of hkv");
  if ((rc = check_qkv_rows(c, rope_len))) return rc;
  const yx::QkvIn in{qkv, q_norm, k_norm, rope_cs, static_cast<uint32_t>(rope_len), eps};
  return qk_rope_impl(c, kv, layer, in, hq, q_out);
}

int yx_attention_qkv_dev(yx_ctx* c, yx_kv* kv, size_t layer, const float* qkv,
                         const float* q_norm, const float* k_norm, const float* rope_cs,
                         size_t rope_len, float eps, float* out, size_t hq, size_t hkv,
                         size_t window, float scale) {
  if (!c || !kv || !qkv || !q_norm || !k_norm || !rope_cs || !out)
    return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  if ((rc = check_kv(c, kv, layer))) return rc;
  if ((rc = check_qkv_rows(c, rope_len))) return rc;
  const yx::QkvIn in{qkv, q_norm, k_norm, rope_cs, static_cast<uint32_t>(rope_len), eps};
  return attention_impl(c, kv, layer, nullptr, out, hq, hkv, window, scale, nullptr, nullptr, &in);
}

int yx_kv_append(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v) {
  if (!c || !kv || !k || !v) return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  const size_t bytes = c->rows * kv->hkv * 128 * 4;
  if ((rc = c->io_a.ensure(std::max<size_t>(bytes, 16), c->stream))) return rc;
  if ((rc = c->io_b.ensure(std::max<size_t>(bytes, 16), c->stream))) return rc;
  YX_HIP(hipMemcpyAsync(c->io_a.p, k, bytes, hipMemcpyHostToDevice, c->stream));
  YX_HIP(hipMemcpyAsync(c->io_b.p, v, bytes, hipMemcpyHostToDevice, c->stream));
  if ((rc = yx_kv_append_dev(c, kv, layer, static_cast<float*>(c->io_a.p), static_cast<float*>(c->io_b.p))))
    return rc;
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_attention_dev(yx_ctx* c, yx_kv* kv, size_t layer, const float* q, float* out, size_t hq,
                     size_t hkv, size_t window, float scale) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  return attention_impl(c, kv, layer, q, out, hq, hkv, window, scale);
}

int yx_attention(yx_ctx* c, yx_kv* kv, size_t layer, const float* q, float* out, size_t hq,
                 size_t hkv, size_t window, float scale) {
  if (!c || !kv || !q || !out) return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  const size_t bytes = c->rows * hq * 128 * 4;
  if ((rc = c->io_a.ensure(std::max<size_t>(bytes, 16), c->stream))) return rc;
  if ((rc = c->io_c.ensure(std::max<size_t>(bytes, 16), c->stream))) return rc;
  YX_HIP(hipMemcpyAsync(c->io_a.p, q, bytes, hipMemcpyHostToDevice, c->stream));
  if ((rc = yx_attention_dev(c, kv, layer, static_cast<float*>(c->io_a.p),
                             static_cast<float*>(c->io_c.p), hq, hkv, window, scale)))
    return rc;
  YX_HIP(hipMemcpyAsync(out, c->io_c.p, bytes, hipMemcpyDeviceToHost, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_attention_append_dev(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v,
                            const float* q, float* out, size_t hq, size_t hkv, size_t window,
                            float scale) {
  if (!c || !kv) return fail(YX_ERR_INVALID, "null argument");
  if (!k || !v) return fail(YX_ERR_INVALID, "null k or v");
  int rc = c->set_device();
  if (rc) return rc;
  return attention_impl(c, kv, layer, q, out, hq, hkv, window, scale, k, v);
}

int yx_attention_append_noalloc(yx_ctx* c, yx_kv* kv, size_t layer, const float* k,
                                const float* v, const float* q, float* out, size_t hq,
                                size_t hkv, size_t window, float scale) {
  if (!c || !kv) return fail(YX_ERR_INVALID, "null argument");
  if (!k || !v) return fail(YX_ERR_INVALID, "null k or v");
  int rc = c->set_device();
  if (rc) return rc;
  return attention_impl(c, kv, layer, q, out, hq, hkv, window, scale, k, v, nullptr, true);
}

int yx_attention_append(yx_ctx* c, yx_kv* kv, size_t layer, const float* k, const float* v,
                        const float* q, float* out, size_t hq, size_t hkv, size_t window,
                        float scale) {
  if (!c || !kv || !k || !v || !q || !out) return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  const size_t qb = c->rows * hq * 128 * 4, kb = c->rows * kv->hkv * 128 * 4;
  if ((rc = c->io_a.ensure(std::max<size_t>(qb, 16), c->stream))) return rc;
  if ((rc = c->io_b.ensure(std::max<size_t>(2 * kb, 16), c->stream))) return rc;
  if ((rc = c->io_c.ensure(std::max<size_t>(qb, 16), c->stream))) return rc;
  float* dk = static_cast<float*>(c->io_b.p);
  float* dv = dk + c->rows * kv->hkv * 128;
  YX_HIP(hipMemcpyAsync(c->io_a.p, q, qb, hipMemcpyHostToDevice, c->stream));
  YX_HIP(hipMemcpyAsync(dk, k, kb, hipMemcpyHostToDevice, c->stream));
  YX_HIP(hipMemcpyAsync(dv, v, kb, hipMemcpyHostToDevice, c->stream));
  if ((rc = yx_attention_append_dev(c, kv, layer, dk, dv, static_cast<float*>(c->io_a.p),
                                    static_cast<float*>(c->io_c.p), hq, hkv, window, scale)))
    return rc;
  YX_HIP(hipMemcpyAsync(out, c->io_c.p, qb, hipMemcpyDeviceToHost, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_dev_alloc(yx_ctx* c, size_t bytes, void** out) {
  if (!c || !out) return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipMalloc(out, std::max<size_t>(bytes, 1)));
  return YX_OK;
}

int yx_dev_free(yx_ctx* c, void* p) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipStreamSynchronize(c->stream));
  if (p) YX_HIP(hipFree(p));
  return YX_OK;
}

int yx_host_alloc(yx_ctx* c, size_t bytes, void** out) {
  if (!c || !out) return fail(YX_ERR_INVALID, "null argument");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipHostMalloc(out, std::max<size_t>(bytes, 1), hipHostMallocDefault));
  return YX_OK;
}

int yx_host_free(yx_ctx* c, void* p) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipStreamSynchronize(c->stream));
  if (p) YX_HIP(hipHostFree(p));
  return YX_OK;
}

int yx_memcpy_h2d(yx_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_memcpy_d2h(yx_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_dev_copy(yx_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  if (bytes && (!dst || !src)) return fail(YX_ERR_INVALID, "null buffer");
  if (bytes % 16 || reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(YX_ERR_INVALID, "dev_copy needs 16-byte aligned sizes and pointers");
  int rc = c->set_device();
  if (rc) return rc;
  const size_t n = bytes / 16;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 8192));
  if (n == 0) return YX_OK;
  hipLaunchKernelGGL(yx::dev_copy16, dim3(blocks), dim3(256), 0, c->stream, static_cast<uint4*>(dst),
                     static_cast<const uint4*>(src), n);
  YX_HIP(hipGetLastError());
  return YX_OK;
}

int yx_dev_checksum(yx_ctx* c, const void* src, size_t bytes, uint64_t* out) {
  if (!c || !out) return fail(YX_ERR_INVALID, "null argument");
  if (bytes && !src) return fail(YX_ERR_INVALID, "null buffer");
  if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(YX_ERR_INVALID, "dev_checksum needs a 16-byte aligned size and pointer");
  int rc = c->set_device();
  if (rc) return rc;
  *out = 0;
  if (bytes == 0) return YX_OK;
  if ((rc = c->io_c.ensure(16, c->stream))) return rc;
  YX_HIP(hipMemsetAsync(c->io_c.p, 0, 8, c->stream));
  const size_t n = bytes / 16;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 8192));
  hipLaunchKernelGGL(yx::dev_checksum16, dim3(blocks), dim3(256), 0, c->stream,
                     static_cast<const uint4*>(src), n, static_cast<unsigned long long*>(c->io_c.p));
  YX_HIP(hipGetLastError());
  YX_HIP(hipMemcpyAsync(out, c->io_c.p, 8, hipMemcpyDeviceToHost, c->stream));
  YX_HIP(hipStreamSynchronize(c->stream));
  return YX_OK;
}

int yx_matmul_bf16_dev(yx_ctx* c, const float* x, const uint16_t* w, float* out, size_t t,
                       size_t k, size_t n) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  if (t == 0 || n == 0) return YX_OK;
  if (!x || !w || !out) return fail(YX_ERR_INVALID, "null x, w or out");
  if (k == 0 || k % 8) return fail(YX_ERR_UNSUPPORTED, "k must be a positive multiple of 8");
  if (t > 0xffffffffu || k > 0xffffffffu || n > 0xffffffffu || (n + 15) / 16 > 0x7fffffff ||
      (t + 15) / 16 > 0xffff)
    return fail(YX_ERR_UNSUPPORTED, "matmul dimensions too large");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
    return fail(YX_ERR_INVALID, "x and w must be 16-byte aligned");
  int rc = c->set_device();
  if (rc) return rc;
  // Workgroups per output tile along k: about two workgroups per CU in all, each wave
  // at least one pass of its loop (kMmSteps steps of 32).
  const size_t tiles = ((n + 15) / 16) * ((t + 15) / 16), steps = (k + 31) / 32;
  size_t ks = std::max<size_t>(1, std::min<size_t>({(2 * static_cast<size_t>(c->cus) + tiles - 1) / tiles,
                                                     steps / (yx::kMmWaves * yx::kMmSteps), 64}));
  if (c->matmul_k_split > 0) ks = std::min<size_t>(static_cast<size_t>(c->matmul_k_split), steps);
  if (ks > 1) {
    if (c->capturing && (c->mm_part.cap < tiles * ks * 1024 || c->mm_counters.cap < tiles * 4 * yx::kCounterStride))
      return fail(YX_ERR_INVALID, "run the call once before capturing it (its scratch is allocated then)");
    if (tiles * ks * 1024 > 0xffffffffu) return fail(YX_ERR_UNSUPPORTED, "matmul dimensions too large");
    if ((rc = c->mm_part.ensure(tiles * ks * 1024, c->stream))) return rc;
    if ((rc = c->mm_counters.ensure(tiles * 4 * yx::kCounterStride, c->stream, true))) return rc;
  }
  hipLaunchKernelGGL(yx::matmul_bf16_rows,
                     dim3(static_cast<unsigned>((n + 15) / 16), static_cast<unsigned>((t + 15) / 16),
                          static_cast<unsigned>(ks)),
                     dim3(64 * yx::kMmWaves), 0, c->stream, x, w, out, static_cast<uint32_t>(t),
                     static_cast<uint32_t>(k), static_cast<uint32_t>(n),
                     static_cast<yx::f32x4*>(c->mm_part.p), static_cast<uint32_t>(c->mm_part.cap),
                     static_cast<uint32_t*>(c->mm_counters.p));
  YX_HIP(hipGetLastError());
  return YX_OK;
}

int yx_argmax_rows_dev(yx_ctx* c, const float* logits, size_t rows, size_t cols, uint32_t* out) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  if (rows == 0) return YX_OK;
  if (!logits || !out) return fail(YX_ERR_INVALID, "null logits or out");
  if (cols == 0) return fail(YX_ERR_INVALID, "empty rows");
  if (rows > 0xffff || cols > 0x7fffffff) return fail(YX_ERR_UNSUPPORTED, "argmax dimensions too large");
  int rc = c->set_device();
  if (rc) return rc;
  // Slices per row: each thread's share of a slice in one pass of its loads
  // (kArgmaxQuads quads), so a slice takes one round trip to memory.
  const size_t per_slice = static_cast<size_t>(yx::kArgmaxThreads) * yx::kArgmaxQuads * 4;
  size_t nsl = std::max<size_t>(1, std::min<size_t>((cols + per_slice - 1) / per_slice, 1024));
  if (c->argmax_slices > 0) nsl = std::min<size_t>(static_cast<size_t>(c->argmax_slices), cols);
  if (c->capturing && (c->am_keys.cap < rows * nsl * 8 || c->am_counters.cap < rows * 4 * yx::kCounterStride))
    return fail(YX_ERR_INVALID, "run the call once before capturing it (its scratch is allocated then)");
  if ((rc = c->am_keys.ensure(rows * nsl * 8, c->stream))) return rc;
  if ((rc = c->am_counters.ensure(rows * 4 * yx::kCounterStride, c->stream, true))) return rc;
  hipLaunchKernelGGL(yx::argmax_rows, dim3(static_cast<unsigned>(nsl), static_cast<unsigned>(rows)),
                     dim3(yx::kArgmaxThreads), 0, c->stream, logits, static_cast<uint32_t>(cols), out,
                     static_cast<unsigned long long*>(c->am_keys.p), static_cast<uint32_t*>(c->am_counters.p));
  YX_HIP(hipGetLastError());
  return YX_OK;
}

int yx_fill_normal(yx_ctx* c, void* dst, size_t n, int dtype, uint64_t seed, uint64_t offset) {
  if (!c || !dst) return fail(YX_ERR_INVALID, "null argument");
  if (dtype != YX_DTYPE_F16 && dtype != YX_DTYPE_F32) return fail(YX_ERR_INVALID, "bad dtype");
  int rc = c->set_device();
  if (rc) return rc;
  if (n == 0) return YX_OK;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(yx::fill_normal, dim3(blocks), dim3(256), 0, c->stream, dst, n,
                     dtype == YX_DTYPE_F16 ? 1 : 0, seed, offset);
  YX_HIP(hipGetLastError());
  return YX_OK;
}

int yx_graph_begin(yx_ctx* c) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  if (c->capturing) return fail(YX_ERR_INVALID, "already capturing");
  if (c->profiling) return fail(YX_ERR_INVALID, "profiling events cannot be captured");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  c->capturing = true;
  return YX_OK;
}

int yx_graph_end(yx_ctx* c) {
  if (!c || !c->capturing) return fail(YX_ERR_INVALID, "not capturing");
  c->capturing = false;
  hipGraph_t g = nullptr;
  YX_HIP(hipStreamEndCapture(c->stream, &g));
  if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
  if (c->graph) (void)hipGraphDestroy(c->graph);
  c->graph = g;
  c->graph_exec = nullptr;
  YX_HIP(hipGraphInstantiate(&c->graph_exec, g, nullptr, nullptr, 0));
  c->graph_epoch = c->epoch;
  c->graph_gens = c->buffer_gens();
  return YX_OK;
}

int yx_graph_launch(yx_ctx* c) {
  if (!c || !c->graph_exec) return fail(YX_ERR_INVALID, "no captured graph");
  if (c->epoch != c->graph_epoch || c->buffer_gens() != c->graph_gens)
    return fail(YX_ERR_INVALID,
                "the pass, an option, an arena or a buffer changed since the graph was captured; "
                "capture it again");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipGraphLaunch(c->graph_exec, c->stream));
  return YX_OK;
}

int yx_timer_start(yx_ctx* c) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  YX_HIP(hipEventRecord(c->t0, c->stream));
  return YX_OK;
}

int yx_timer_stop(yx_ctx* c, float* ms) {
  if (!c || !ms) return fail(YX_ERR_INVALID, "null argument");
  YX_HIP(hipEventRecord(c->t1, c->stream));
  YX_HIP(hipEventSynchronize(c->t1));
  YX_HIP(hipEventElapsedTime(ms, c->t0, c->t1));
  return YX_OK;
}

int yx_profile_enable(yx_ctx* c, int on) {
  if (!c) return fail(YX_ERR_INVALID, "null context");
  c->profiling = on != 0;
  return YX_OK;
}

int yx_profile_read(yx_ctx* c, int kernel, double* total_ms, uint64_t* launches) {
  if (!c || kernel < 0 || kernel > 3) return fail(YX_ERR_INVALID, "bad context or kernel");
  int rc = c->set_device();
  if (rc) return rc;
  YX_HIP(hipStreamSynchronize(c->stream));
  Profile& p = c->prof[kernel];
  for (auto& e : p.pending) {
    float ms = 0;
    YX_HIP(hipEventElapsedTime(&ms, e.first, e.second));
    p.total_ms += ms;
    p.launches += 1;
    (void)hipEventDestroy(e.first);
    (void)hipEventDestroy(e.second);
  }
  p.pending.clear();
  if (total_ms) *total_ms = p.total_ms;
  if (launches) *launches = p.launches;
  p.total_ms = 0;
  p.launches = 0;
  return YX_OK;
}

}  // extern "C"
