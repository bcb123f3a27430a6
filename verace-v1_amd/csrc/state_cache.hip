// Decode state cache: per-layer pools of SSSD states with copy-on-write branches, and
// the batched decode step over them (extern "C" entry points vmi_state_cache_*,
// declared in include/verace_sssd.h).
//
// The reference keeps decode state as Python lists, layer_states[l][i] =
// (sssd_state, cham_hologram) (acd_engine.py:85-126), steps the batch one item at a
// time, and forks tree-search branches by copying those lists so that every candidate
// token starts from the same cached state (hyper_generate.py:97-121).  Here the caller
// allocates one device pool [L, N, H, D, D] fp32 and this object keeps, on the host:
//   phys[h][l]  the slot holding handle h's state at layer l (-1: still the identity)
//   refs[l][s]  how many handles hold slot s of layer l; a free stack per layer.
// A step of layer l over a list of handles is one launch of the decode-step kernel with
// the slot of every item passed in the kernel arguments (SlotArgs, no device array and no
// host-to-device copy).  A handle that is its slot's only holder is updated in place;
// a handle that shares its slot (after a fork) or has none reads the shared slot (or
// the identity) and writes a fresh one, so copy-on-write costs no extra pass over the
// state.  Decisions use the reference counts from before the step and all fresh slots
// are taken before any slot is freed, so within one launch every written slot is
// distinct and is read by no other item.
//
// The object holds host memory only; the pool is the caller's.  It is not thread-safe:
// one host thread drives a cache.  Launches go to the stream given to each step, and
// slot reuse relies on the steps of a cache being ordered (one stream).
#include <vector>

#include "vmi_common.h"
#include "vmi_dispatch.h"

struct vmi_state_cache {
  int64_t L = 0, N = 0, H = 0, D = 0;
  float* pool = nullptr;
  std::vector<int32_t> refs;                  // [L * N]
  std::vector<std::vector<int32_t>> free;     // per layer, LIFO (a freed slot is reused first)
  std::vector<std::vector<int32_t>> phys;     // per handle id: [L], empty once released
  std::vector<int64_t> free_ids;              // released handle ids, reused LIFO
  std::vector<uint64_t> mark;                 // per handle id: stamp of the last call seen
  uint64_t stamp = 0;
  // scratch of the last plan (host)
  std::vector<int32_t> src, dst;
  std::vector<char> inplace;
  // the CHAM half of each layer's state (vmi_state_cache_attach_hologram): pool
  // [L, N, 2, h, h] fp32, slot s of layer l at holo + (l N + s) 2 h^2; the hologram of a
  // handle lives in the same slot as its SSSD state, and a layer's CHAM step applies the
  // slot decisions of that layer's last SSSD step (same handles, same order)
  int64_t h = 0;
  float* holo = nullptr;
  std::vector<std::vector<int64_t>> last_handles;  // per layer
  std::vector<std::vector<int32_t>> last_src, last_dst;
};

namespace {

bool valid_handle(const vmi_state_cache* c, int64_t h) {
  return h >= 0 && h < static_cast<int64_t>(c->phys.size()) && !c->phys[h].empty();
}

int64_t new_handle(vmi_state_cache* c) {
  int64_t h;
  if (!c->free_ids.empty()) {
    h = c->free_ids.back();
    c->free_ids.pop_back();
  } else {
    h = static_cast<int64_t>(c->phys.size());
    c->phys.emplace_back();
    c->mark.push_back(0);
  }
  c->phys[h].assign(c->L, -1);
  return h;
}

// Slot decisions recorded for the CHAM half hold only until the table changes: a fork
// adds holders to slots, a release frees them for reuse.
void forget_cham_decisions(vmi_state_cache* c) {
  for (auto& lh : c->last_handles) lh.clear();
}

void unref(vmi_state_cache* c, int64_t l, int32_t s) {
  int32_t& r = c->refs[l * c->N + s];
  if (--r == 0) c->free[l].push_back(s);
}

// Validates a handle list: every handle live, none repeated within the call.
bool check_handles(vmi_state_cache* c, const int64_t* handles, int64_t n) {
  if (n > 0 && handles == nullptr) return false;
  ++c->stamp;
  for (int64_t b = 0; b < n; ++b) {
    const int64_t h = handles[b];
    if (!valid_handle(c, h) || c->mark[h] == c->stamp) return false;
    c->mark[h] = c->stamp;
  }
  return true;
}

// Plans one step (or one whole-state write) of layer l over handles[0..n): fills c->src /
// c->dst and updates the table as if it had run.
int plan(vmi_state_cache* c, int64_t l, const int64_t* handles, int64_t n) {
  if (l < 0 || l >= c->L || n < 0) return VMI_ERR_INVALID_ARG;
  c->last_handles[l].clear();  // any new plan of the layer voids the recorded CHAM decisions
  if (!check_handles(c, handles, n)) return VMI_ERR_INVALID_ARG;
  c->src.resize(n);
  c->dst.resize(n);
  c->inplace.resize(n);
  int64_t need = 0;
  for (int64_t b = 0; b < n; ++b) {
    const int32_t s = c->phys[handles[b]][l];
    c->src[b] = s;
    c->inplace[b] = s >= 0 && c->refs[l * c->N + s] == 1;
    need += !c->inplace[b];
  }
  if (need > static_cast<int64_t>(c->free[l].size())) return VMI_ERR_FULL;
  // take every fresh slot before freeing any, so none is both read and written here
  for (int64_t b = 0; b < n; ++b) {
    if (c->inplace[b]) {
      c->dst[b] = c->src[b];
    } else {
      const int32_t s = c->free[l].back();
      c->free[l].pop_back();
      c->refs[l * c->N + s] = 1;
      c->dst[b] = s;
    }
  }
  for (int64_t b = 0; b < n; ++b) {
    if (c->inplace[b]) continue;
    if (c->src[b] >= 0) unref(c, l, c->src[b]);
    c->phys[handles[b]][l] = c->dst[b];
  }
  return VMI_OK;
}

}  // namespace

extern "C" {

int vmi_state_cache_create(int64_t num_layers, int64_t num_slots, int64_t H, int64_t D,
                           float* pool, vmi_state_cache** cache) {
  if (cache == nullptr) return VMI_ERR_INVALID_ARG;
  *cache = nullptr;
  if (num_layers < 1 || num_slots < 1 || num_slots > INT32_MAX || H < 1 || D < 1)
    return VMI_ERR_INVALID_ARG;
  if (D > 256) return VMI_ERR_UNSUPPORTED;
  vmi_state_cache* c = new vmi_state_cache;
  c->L = num_layers;
  c->N = num_slots;
  c->H = H;
  c->D = D;
  c->pool = pool;
  c->refs.assign(num_layers * num_slots, 0);
  c->last_handles.resize(num_layers);
  c->last_src.resize(num_layers);
  c->last_dst.resize(num_layers);
  c->free.resize(num_layers);
  for (auto& f : c->free)
    for (int64_t s = num_slots - 1; s >= 0; --s) f.push_back(static_cast<int32_t>(s));
  *cache = c;
  return VMI_OK;
}

int vmi_state_cache_destroy(vmi_state_cache* cache) {
  delete cache;
  return VMI_OK;
}

int vmi_state_cache_new(vmi_state_cache* c, int64_t n, int64_t* handles) {
  if (c == nullptr || n < 0 || (n > 0 && handles == nullptr)) return VMI_ERR_INVALID_ARG;
  for (int64_t i = 0; i < n; ++i) handles[i] = new_handle(c);
  return VMI_OK;
}

int vmi_state_cache_fork(vmi_state_cache* c, int64_t parent, int64_t n, int64_t* handles) {
  if (c == nullptr || n < 0 || (n > 0 && handles == nullptr)) return VMI_ERR_INVALID_ARG;
  if (!valid_handle(c, parent)) return VMI_ERR_INVALID_ARG;
  if (n > 0) forget_cham_decisions(c);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t h = new_handle(c);  // may grow phys: index the parent afresh
    c->phys[h] = c->phys[parent];
    for (int64_t l = 0; l < c->L; ++l)
      if (c->phys[h][l] >= 0) ++c->refs[l * c->N + c->phys[h][l]];
    handles[i] = h;
  }
  return VMI_OK;
}

int vmi_state_cache_release(vmi_state_cache* c, const int64_t* handles, int64_t n) {
  if (c == nullptr || n < 0 || !check_handles(c, handles, n)) return VMI_ERR_INVALID_ARG;
  if (n > 0) forget_cham_decisions(c);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t h = handles[i];
    for (int64_t l = 0; l < c->L; ++l)
      if (c->phys[h][l] >= 0) unref(c, l, c->phys[h][l]);
    c->phys[h].clear();
    c->free_ids.push_back(h);
  }
  return VMI_OK;
}

int vmi_state_cache_plan(vmi_state_cache* c, int64_t layer, const int64_t* handles, int64_t n,
                         int32_t* src, int32_t* dst) {
  if (c == nullptr) return VMI_ERR_INVALID_ARG;
  const int st = plan(c, layer, handles, n);
  if (st != VMI_OK) return st;
  for (int64_t b = 0; b < n; ++b) {
    if (src != nullptr) src[b] = c->src[b];
    if (dst != nullptr) dst[b] = c->dst[b];
  }
  return VMI_OK;
}

int vmi_state_cache_slots(vmi_state_cache* c, int64_t layer, const int64_t* handles, int64_t n,
                          int32_t* slots) {
  if (c == nullptr || layer < 0 || layer >= c->L || n < 0 || (n > 0 && slots == nullptr))
    return VMI_ERR_INVALID_ARG;
  if (!check_handles(c, handles, n)) return VMI_ERR_INVALID_ARG;
  for (int64_t b = 0; b < n; ++b) slots[b] = c->phys[handles[b]][layer];
  return VMI_OK;
}

int vmi_state_cache_refs(vmi_state_cache* c, int64_t layer, int32_t* refs, int64_t* free_slots) {
  if (c == nullptr || layer < 0 || layer >= c->L) return VMI_ERR_INVALID_ARG;
  if (refs != nullptr)
    for (int64_t s = 0; s < c->N; ++s) refs[s] = c->refs[layer * c->N + s];
  if (free_slots != nullptr) *free_slots = static_cast<int64_t>(c->free[layer].size());
  return VMI_OK;
}

int vmi_state_cache_step(vmi_state_cache* c, int64_t layer, const int64_t* handles, int64_t n,
                         const void* q, const void* k, const void* v, const void* delta,
                         int io_dtype, int delta_dtype, void* out, void* stream) {
  if (c == nullptr) return VMI_ERR_INVALID_ARG;
  if (io_dtype != VMI_F32 && io_dtype != VMI_BF16 && io_dtype != VMI_F16) return VMI_ERR_INVALID_ARG;
  if (delta_dtype != VMI_F32 && delta_dtype != VMI_BF16 && delta_dtype != VMI_F16)
    return VMI_ERR_INVALID_ARG;
  if (n > 0 && (q == nullptr || k == nullptr || v == nullptr || delta == nullptr ||
                out == nullptr || c->pool == nullptr))
    return VMI_ERR_INVALID_ARG;
  if (n * c->H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  const int st = plan(c, layer, handles, n);
  if (st != VMI_OK) return st;
  c->last_handles[layer].assign(handles, handles + n);
  c->last_src[layer] = c->src;
  c->last_dst[layer] = c->dst;
  const int64_t H = c->H, D = c->D;
  const size_t io_bytes = io_dtype == VMI_F32 ? 4 : 2;
  const size_t d_bytes = delta_dtype == VMI_F32 ? 4 : 2;
  float* pool = c->pool + layer * c->N * H * D * D;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // batches above kMaxSlotArgs items go out as several launches on the same stream
  for (int64_t b0 = 0; b0 < n; b0 += vmi::kMaxSlotArgs) {
    const int nb = static_cast<int>(n - b0 < vmi::kMaxSlotArgs ? n - b0 : vmi::kMaxSlotArgs);
    vmi::SlotArgs map;
    map.nslots = static_cast<int>(c->N);
    for (int i = 0; i < nb; ++i) {
      map.in_slot[i] = c->src[b0 + i];
      map.out_slot[i] = c->dst[b0 + i];
    }
    const size_t tok = static_cast<size_t>(b0) * H * D * io_bytes;
    const char* qb = static_cast<const char*>(q) + tok;
    const char* kb = static_cast<const char*>(k) + tok;
    const char* vb = static_cast<const char*>(v) + tok;
    char* ob = static_cast<char*>(out) + tok;
    const char* db = static_cast<const char*>(delta) + static_cast<size_t>(b0) * H * d_bytes;
    hipError_t e;
    if (vmi::use_step128(1, D))
      e = vmi::launch_sssd_step128(qb, kb, vb, db, io_dtype, delta_dtype, pool, ob, pool, map, nb,
                                   static_cast<int>(H), s);
    else
      e = vmi::launch_sssd_seq(qb, kb, vb, db, io_dtype, delta_dtype, pool, ob, pool, nb, 1,
                               static_cast<int>(H), static_cast<int>(D), s, map);
    if (e != hipSuccess) return vmi::hip_status(e);
  }
  return VMI_OK;
}

int vmi_state_cache_attach_hologram(vmi_state_cache* c, int64_t h, float* holo_pool) {
  if (c == nullptr || h < 1 || holo_pool == nullptr) return VMI_ERR_INVALID_ARG;
  if (h > 1024 || h % 4 != 0) return VMI_ERR_UNSUPPORTED;
  c->h = h;
  c->holo = holo_pool;
  return VMI_OK;
}

int vmi_state_cache_cham_workspace_bytes(int64_t n, int64_t h, size_t* bytes) {
  if (bytes == nullptr || n < 0 || h < 1) return VMI_ERR_INVALID_ARG;
  const int64_t nb = n < vmi::kMaxSlotArgs ? n : vmi::kMaxSlotArgs;
  *bytes = vmi::cham_step_workspace_bytes(nb, h);
  return VMI_OK;
}

int vmi_state_cache_cham_step(vmi_state_cache* c, int64_t layer, const int64_t* handles,
                              int64_t n, const void* q, const void* k, const void* v,
                              const void* gamma, int io_dtype, int gamma_dtype, void* out,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (c == nullptr || c->holo == nullptr || layer < 0 || layer >= c->L || n < 0)
    return VMI_ERR_INVALID_ARG;
  if (io_dtype != VMI_F32 && io_dtype != VMI_BF16 && io_dtype != VMI_F16) return VMI_ERR_INVALID_ARG;
  if (gamma_dtype != VMI_F32 && gamma_dtype != VMI_BF16 && gamma_dtype != VMI_F16)
    return VMI_ERR_INVALID_ARG;
  // the same handles, in the same order, as this layer's last SSSD step, once, with no
  // fork, release or other plan of the layer in between
  auto& lh = c->last_handles[layer];
  if (static_cast<int64_t>(lh.size()) != n) return VMI_ERR_INVALID_ARG;
  for (int64_t b = 0; b < n; ++b)
    if (handles == nullptr || lh[b] != handles[b]) return VMI_ERR_INVALID_ARG;
  if (n == 0) {
    lh.clear();
    return VMI_OK;
  }
  if (q == nullptr || k == nullptr || v == nullptr || gamma == nullptr || out == nullptr)
    return VMI_ERR_INVALID_ARG;
  size_t need = 0;
  vmi_state_cache_cham_workspace_bytes(n, c->h, &need);
  if (workspace == nullptr || workspace_bytes < need) return VMI_ERR_WORKSPACE;
  const int64_t h = c->h;
  const size_t io_bytes = io_dtype == VMI_F32 ? 4 : 2;
  const size_t g_bytes = gamma_dtype == VMI_F32 ? 4 : 2;
  float* pool = c->holo + layer * c->N * 2 * h * h;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int64_t b0 = 0; b0 < n; b0 += vmi::kMaxSlotArgs) {
    const int nb = static_cast<int>(n - b0 < vmi::kMaxSlotArgs ? n - b0 : vmi::kMaxSlotArgs);
    const size_t tok = static_cast<size_t>(b0) * h * io_bytes;
    const hipError_t e = vmi::launch_cham_step_slots(
        static_cast<const char*>(q) + tok, static_cast<const char*>(k) + tok,
        static_cast<const char*>(v) + tok, static_cast<const char*>(gamma) + b0 * g_bytes, io_dtype,
        gamma_dtype, pool, c->last_src[layer].data() + b0, c->last_dst[layer].data() + b0,
        static_cast<char*>(out) + tok, nb, static_cast<int>(h), workspace, s);
    if (e != hipSuccess) {
      lh.clear();
      return vmi::hip_status(e);
    }
  }
  lh.clear();  // the decisions are spent: a second call would copy into in-place slots
  return VMI_OK;
}

}  // extern "C"
