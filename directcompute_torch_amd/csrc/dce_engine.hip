// libdcengine: device, buffer pool, dispatch registry and the fused C entry
// points of the engine.dll ABI (include/dcengine.h), on one HIP stream.
//
// Design notes
//  * One in-order stream replaces the D3D11 immediate context: a buffer that
//    the host releases to the pool and hands out again is only touched by
//    work queued after every earlier user, so pooled reuse needs no fences.
//  * Device memory is freed only after the stream has drained.
//  * Host->device copies never block on queued work: payloads of up to 256
//    floats travel as kernel arguments, larger ones through a ring of pinned
//    staging slots guarded by events.
#include "dce_internal.h"
#include "../../include/dcengine.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

namespace dce {

// ---------------------------------------------------------------------------
// Global state
// ---------------------------------------------------------------------------
static bool g_init = false;
static int g_device = 0;
static hipStream_t g_stream = nullptr;
static int g_cus = 256;
static GPUInfo g_info;
static char g_err[1024] = "";

static std::unordered_map<uint32_t, std::vector<Buffer*>> g_pool;
static std::vector<Buffer*> g_recycled;  // dead records, reused for new handles
static uint64_t g_poolHits = 0, g_poolMisses = 0, g_poolBytes = 0;
static uint64_t g_poolCapBytes = 0;

double g_streamBytes = kStreamBytes;

static float* g_ws = nullptr;
static size_t g_wsFloats = 0;

// HIP-graph capture of the engine stream (BeginCapture / EndCapture).  While a
// capture is open every buffer handed out or released is held for the graph
// (a recorded node may read it), nothing is freed, and calls that would wait
// on the stream are refused.  Workspace
// blocks a live graph may reference are retired, not freed.
static bool g_capturing = false;
static bool g_captureFailed = false;
static std::vector<Buffer*> g_captureHeld;
static std::vector<float*> g_wsRetired;
static int g_liveGraphs = 0;
static bool refuse_in_capture(const char* what);
static float* g_misc = nullptr;  // 1024 floats of device scratch for scalars
static float* g_ones = nullptr;  // 4 floats of 1.0

// Pinned staging ring for host->device uploads.
constexpr int kSlots = 4;
constexpr size_t kSlotBytes = size_t(16) << 20;
static char* g_stage = nullptr;
static hipEvent_t g_slotEv[kSlots];
static bool g_slotBusy[kSlots];
static int g_nextSlot = 0;

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

hipStream_t stream() { return g_stream; }
const float* ones4() { return g_ones; }
int num_cus() { return g_cus; }

bool ensure_init() {
  if (g_init) return true;
  set_error("engine not initialised (InitEngine failed or was not called)");
  return false;
}

// Calls that wait on the stream (or stage host memory) cannot be recorded:
// during a capture they fail, and the capture is marked failed so that
// EndCapture returns NULL with this reason.
static bool refuse_in_capture(const char* what) {
  if (!g_capturing) return false;
  set_error("%s is not allowed while a graph capture is open", what);
  g_captureFailed = true;
  return true;
}

bool check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return false;
  }
  return true;
}

int blocks_per_cu_raw(const void* kernel, int threads) {
  static std::map<std::pair<const void*, int>, int> cache;
  const auto key = std::make_pair(kernel, threads);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1) {
    hipGetLastError();
    n = 1;
  }
  cache[key] = n;
  return n;
}

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d ? d : 1;
  uint32_t l = 0;
  while ((uint64_t(1) << l) < f.d) ++l;
  uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - f.d)) / f.d + 1;
  f.mul = uint32_t(m);
  f.shr = l;
  return f;
}

// ---------------------------------------------------------------------------
// Profiling: per-family event timing on the engine stream.
// ---------------------------------------------------------------------------
struct ProfStat {
  uint64_t launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};
struct ProfPending {
  const char* family;
  hipEvent_t e0, e1;
  double flops, bytes;
};
static bool g_prof = false;
static std::unordered_map<std::string, ProfStat> g_profStats;
static std::vector<ProfPending> g_profPending;
static std::vector<hipEvent_t> g_eventFree;

static hipEvent_t take_event() {
  if (!g_eventFree.empty()) {
    hipEvent_t e = g_eventFree.back();
    g_eventFree.pop_back();
    return e;
  }
  // Timing only: no system-scope fence when the event is recorded (the
  // fence writes back and invalidates the caches, which cost every profiled
  // launch a cold L2 and a few microseconds of idle GPU).  The profile is
  // read after a stream synchronisation.
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

// Families recorded while profiling is on (empty: all).
static std::vector<std::string> g_profFilter;
static bool prof_wanted(const char* fam) {
  if (g_profFilter.empty()) return true;
  for (const std::string& f : g_profFilter)
    if (f == fam) return true;
  return false;
}

ProfScope::ProfScope(const char* fam, double fl, double by)
    : family(fam), flops(fl), bytes(by), ev0(nullptr) {
  if (!g_prof || g_capturing || !prof_wanted(fam)) return;
  hipEvent_t e = take_event();
  if (!e) return;
  hipEventRecord(e, g_stream);
  ev0 = e;
}

ProfScope::~ProfScope() {
  if (!ev0) return;
  hipEvent_t e1 = take_event();
  if (!e1) return;
  hipEventRecord(e1, g_stream);
  g_profPending.push_back({family, (hipEvent_t)ev0, e1, flops, bytes});
}

static void resolve_profile() {
  if (g_profPending.empty() || g_capturing) return;
  hipStreamSynchronize(g_stream);
  for (auto& p : g_profPending) {
    float ms = 0;
    hipEventElapsedTime(&ms, p.e0, p.e1);
    ProfStat& s = g_profStats[p.family];
    s.launches++;
    s.ms += ms;
    s.flops += p.flops;
    s.bytes += p.bytes;
    g_eventFree.push_back(p.e0);
    g_eventFree.push_back(p.e1);
  }
  g_profPending.clear();
}

// ---------------------------------------------------------------------------
// Buffers and pool
// ---------------------------------------------------------------------------
// Copies of one size the pool keeps.  The real bound is the byte cap (half of
// device memory): a step that holds dozens of same-size activations at once
// (UNet or MobileNet at full resolution) gets all of them back next step,
// instead of freeing the excess (a stream drain each) and allocating again.
static size_t max_pool_for_size(uint32_t) { return 4096; }

// Producer tags (Buffer::tag).  A new tag gets a fresh generation; dropping
// one releases the buffer it owns.
static uint64_t g_gen = 0;
static void set_tag(Buffer* b, uint32_t tag) {
  b->tag = tag;
  b->gen = ++g_gen;
}
// park: the owned buffer goes back to the pool even past the pool's byte
// cap, so that the call frees nothing (the no-allocation entry point).
static void park_buffer(Buffer* b);
static void drop_tag(Buffer* b, bool park = false) {
  b->tag = 0;
  b->src = b->aux = nullptr;
  b->key = nullptr;
  if (Buffer* s = b->side) {
    b->side = nullptr;
    if (park) park_buffer(s); else release_buffer(s);
  }
}
void tag_bn_stats(void* y, void* side, uint32_t B, uint32_t C, uint32_t S, uint32_t pieces,
                  uint32_t H, uint32_t W) {
  Buffer* Y = static_cast<Buffer*>(y);
  if (!Y || Y->magic != kMagicLive) {
    release_buffer(side);
    return;
  }
  drop_tag(Y);
  set_tag(Y, kBnStatsTag);
  Y->meta[0] = B;
  Y->meta[1] = C;
  Y->meta[2] = S;
  Y->meta[3] = H;
  Y->meta[4] = W;
  Y->aux32 = pieces;
  Y->side = static_cast<Buffer*>(side);
}
// The activation that followed each batch norm (keyed by its gamma buffer
// record) the last time one ran on its output.
static std::unordered_map<const void*, uint32_t> g_bnAct;
uint32_t bn_act_guess(const void* gamma) {
  auto it = gamma ? g_bnAct.find(gamma) : g_bnAct.end();
  return it == g_bnAct.end() ? 0u : it->second;
}
void tag_bn_out(void* z, void* x, void* mean, void* gamma, void* side, uint32_t act,
                uint32_t N, uint32_t C, uint32_t S, float eps) {
  Buffer* Z = static_cast<Buffer*>(z);
  if (!Z || Z->magic != kMagicLive) {
    release_buffer(side);
    return;
  }
  drop_tag(Z);
  set_tag(Z, kBnOutTag);
  Z->key = gamma;
  Z->aux32 = side ? act : 0u;
  Z->side = static_cast<Buffer*>(side);
  Z->meta[0] = N;
  Z->meta[1] = C;
  Z->meta[2] = S;
  memcpy(&Z->aux32b, &eps, 4);
  // x and the statistics, linked while they carry the tags they have now
  // (the backward's fused reduce uses them only then).
  Buffer* X = static_cast<Buffer*>(x);
  Buffer* M = static_cast<Buffer*>(mean);
  if (X && X->magic == kMagicLive && X->tag == kBnStatsTag && M && M->magic == kMagicLive &&
      M->tag == kBnMomentTag) {
    Z->src = X;
    Z->srcGen = X->gen;
    Z->aux = M;
    Z->auxGen = M->gen;
  }
}
void tag_bn_moments(void* mean, void* var) {
  Buffer* M = static_cast<Buffer*>(mean);
  Buffer* V = static_cast<Buffer*>(var);
  if (!M || !V || M == V || M->magic != kMagicLive || V->magic != kMagicLive) return;
  drop_tag(V);
  set_tag(V, kBnMomentTag);
  drop_tag(M);
  set_tag(M, kBnMomentTag);
  M->src = V;
  M->srcGen = V->gen;
}
// z's batch norm operands, each still carrying the tag it had when linked.
static bool bn_links_alive(const Buffer* Z, Buffer** x, Buffer** mean, Buffer** var) {
  if (!Z || Z->magic != kMagicLive || Z->tag != kBnOutTag || !Z->src || !Z->aux) return false;
  Buffer* X = Z->src;
  Buffer* M = Z->aux;
  if (!tag_alive(X, kBnStatsTag, Z->srcGen) || !tag_alive(M, kBnMomentTag, Z->auxGen) ||
      !tag_alive(M->src, kBnMomentTag, M->srcGen))
    return false;
  *x = X;
  *mean = M;
  *var = M->src;
  return true;
}
bool bn_link_of(void* z, BnLink* out) {
  const Buffer* Z = static_cast<const Buffer*>(z);
  Buffer *X, *M, *V;
  if (!bn_links_alive(Z, &X, &M, &V)) return false;
  const uint64_t n = uint64_t(Z->meta[0]) * Z->meta[1] * Z->meta[2];
  if (X->count < n || Z->count < n || M->count < Z->meta[1] || V->count < Z->meta[1]) return false;
  out->x = X->ptr;
  out->mean = M->ptr;
  out->var = V->ptr;
  out->N = Z->meta[0];
  out->C = Z->meta[1];
  out->S = Z->meta[2];
  memcpy(&out->eps, &Z->aux32b, 4);
  return true;
}
void tag_bn_grad_part(void* dz, void* z, void* side, uint32_t pieces) {
  Buffer* D = static_cast<Buffer*>(dz);
  const Buffer* Z = static_cast<const Buffer*>(z);
  Buffer *X, *M, *V;
  if (!D || D->magic != kMagicLive || !bn_links_alive(Z, &X, &M, &V)) {
    release_buffer(side);
    return;
  }
  drop_tag(D);
  set_tag(D, kBnGradPartTag);
  D->side = static_cast<Buffer*>(side);
  D->src = X;
  D->srcGen = X->gen;
  D->aux = M;
  D->auxGen = M->gen;
  for (int i = 0; i < 3; ++i) D->meta[i] = Z->meta[i];
  D->aux32 = pieces;
  D->aux32b = Z->aux32b;
}
const double* bn_grad_part_of(void* dy, void* x, void* mean, void* var, uint32_t N, uint32_t C,
                              uint32_t S, float eps, uint32_t* pieces) {
  const Buffer* D = static_cast<const Buffer*>(dy);
  if (!D || D->magic != kMagicLive || D->tag != kBnGradPartTag || !D->side) return nullptr;
  uint32_t eb;
  memcpy(&eb, &eps, 4);
  Buffer* M = D->aux;
  if (D->src != x || M != mean || !tag_alive(D->src, kBnStatsTag, D->srcGen) ||
      !tag_alive(M, kBnMomentTag, D->auxGen) || M->src != var ||
      !tag_alive(M->src, kBnMomentTag, M->srcGen) || D->meta[0] != N || D->meta[1] != C ||
      D->meta[2] != S || D->aux32b != eb)
    return nullptr;
  *pieces = D->aux32;
  return reinterpret_cast<const double*>(D->side->ptr);
}
bool bn_act_adopt(void* z, void* a, uint32_t act, uint32_t n) {
  Buffer* Z = static_cast<Buffer*>(z);
  Buffer* A = static_cast<Buffer*>(a);
  if (!Z || Z->magic != kMagicLive || Z->tag != kBnOutTag) return false;
  if (Z->key) g_bnAct[Z->key] = act;
  Buffer* S = Z->side;
  if (!S || Z->aux32 != act || !A || A == Z || A->magic != kMagicLive || A->count != S->count ||
      n != S->count)
    return false;
  // A's contents become act(z): take S's storage, give S A's (same size) and
  // return S to the pool.  Handles are opaque, so no caller holds the old
  // address; work already queued on A's old storage runs before any reuse
  // (one stream).
  std::swap(A->ptr, S->ptr);
  Z->side = nullptr;
  Z->aux32 = 0;
  release_buffer(S);
  return true;
}

void tag_grad_g_nhwc(void* dx, void* side, uint32_t B, uint32_t C, uint32_t H, uint32_t W,
                     uint32_t rows) {
  Buffer* D = static_cast<Buffer*>(dx);
  if (!D || D->magic != kMagicLive) {
    release_buffer(side);
    return;
  }
  drop_tag(D);
  set_tag(D, kGradGTag);
  D->meta[0] = kGLayoutNhwc;
  D->meta[1] = B;
  D->meta[2] = C;
  D->meta[3] = H;
  D->meta[4] = W;
  D->aux32 = rows;
  D->side = static_cast<Buffer*>(side);
}

// Buffers an entry point writes in place lose their tags.
static void drop_tags(void** hs, uint32_t n, bool park = false) {
  for (uint32_t i = 0; hs && i < n; ++i) {
    Buffer* b = static_cast<Buffer*>(hs[i]);
    if (b && b->magic == kMagicLive) drop_tag(b, park);
  }
}

static void free_record(Buffer* b) {
  // The stream may still reference the memory: drain it first.
  hipStreamSynchronize(g_stream);
  hipFree(b->ptr);
  b->ptr = nullptr;
  b->magic = kMagicDead;
  b->refCount = 0;
  g_recycled.push_back(b);
}

static void drain_pool_locked() {
  if (g_capturing) return;  // frees would wait on the stream
  bool any = false;
  for (auto& kv : g_pool) any |= !kv.second.empty();
  if (!any) return;
  hipStreamSynchronize(g_stream);
  for (auto& kv : g_pool) {
    for (Buffer* b : kv.second) {
      hipFree(b->ptr);
      b->ptr = nullptr;
      b->magic = kMagicDead;
      g_recycled.push_back(b);
    }
    kv.second.clear();
  }
  g_pool.clear();
  g_poolBytes = 0;
}

Buffer* as_buffer(void* h, const char* what) {
  if (!h) {
    set_error("%s: NULL buffer handle", what);
    return nullptr;
  }
  Buffer* b = static_cast<Buffer*>(h);
  if (b->magic != kMagicLive) {
    set_error("%s: handle %p is not a live buffer (released or foreign)", what, h);
    return nullptr;
  }
  return b;
}

// Small uploads travel as kernel arguments: the launch copies them, so the
// host memory is free on return and nothing waits for queued work.
struct SmallPayload {
  float v[256];
};
__global__ void k_upload_small(float* __restrict__ dst, SmallPayload pl, uint32_t n) {
  uint32_t i = threadIdx.x;
  if (i < n) dst[i] = pl.v[i];
}

static bool upload(float* dst, const float* src, size_t n) {
  if (n == 0) return true;
  if (n <= 256) {
    SmallPayload pl;
    memcpy(pl.v, src, n * 4);
    hipLaunchKernelGGL(k_upload_small, dim3(1), dim3(256), 0, g_stream, dst, pl, uint32_t(n));
    return check_launch("upload");
  }
  // A staged copy would replay whatever the staging slot holds later.
  if (refuse_in_capture("a host upload of more than 256 floats")) return false;
  if (!g_stage) {
    if (hipHostMalloc((void**)&g_stage, kSlots * kSlotBytes, hipHostMallocDefault) != hipSuccess) {
      g_stage = nullptr;
      set_error("upload: pinned staging allocation failed");
      return false;
    }
    for (int i = 0; i < kSlots; ++i) {
      hipEventCreateWithFlags(&g_slotEv[i], hipEventDisableTiming);
      g_slotBusy[i] = false;
    }
  }
  const char* s = reinterpret_cast<const char*>(src);
  char* d = reinterpret_cast<char*>(dst);
  size_t bytes = n * 4;
  while (bytes) {
    size_t chunk = std::min(bytes, kSlotBytes);
    int slot = g_nextSlot;
    g_nextSlot = (g_nextSlot + 1) % kSlots;
    if (g_slotBusy[slot]) hipEventSynchronize(g_slotEv[slot]);
    char* st = g_stage + size_t(slot) * kSlotBytes;
    memcpy(st, s, chunk);
    if (hipMemcpyAsync(d, st, chunk, hipMemcpyHostToDevice, g_stream) != hipSuccess) {
      set_error("upload: hipMemcpyAsync failed");
      return false;
    }
    hipEventRecord(g_slotEv[slot], g_stream);
    g_slotBusy[slot] = true;
    s += chunk;
    d += chunk;
    bytes -= chunk;
  }
  return true;
}

// A fresh device allocation (never from the pool), refcount 1.
static Buffer* alloc_record(uint32_t count) {
  float* p = nullptr;
  const size_t bytes = size_t(count) * 4;
  if (hipMalloc((void**)&p, bytes) != hipSuccess) {
    hipGetLastError();
    drain_pool_locked();
    if (hipMalloc((void**)&p, bytes) != hipSuccess) {
      hipGetLastError();
      set_error("CreateBuffer: out of device memory for %u floats", count);
      return nullptr;
    }
  }
  Buffer* b = nullptr;
  if (!g_recycled.empty()) {
    b = g_recycled.back();
    g_recycled.pop_back();
  } else {
    b = new Buffer();
  }
  b->ptr = p;
  b->count = count;
  b->refCount = 1;
  b->magic = kMagicLive;
  b->tag = 0;
  b->gen = 0;
  b->src = b->aux = b->side = nullptr;
  b->key = nullptr;
  return b;
}

void* create_buffer(const float* data, uint32_t count) {
  if (!ensure_init()) return nullptr;
  if (count == 0) {
    set_error("CreateBuffer: zero-size buffer");
    return nullptr;
  }
  Buffer* b = nullptr;
  auto it = g_pool.find(count);
  if (it != g_pool.end() && !it->second.empty()) {
    b = it->second.back();
    it->second.pop_back();
    g_poolBytes -= uint64_t(count) * 4;
    g_poolHits++;
    b->refCount = 1;
    b->magic = kMagicLive;
    b->tag = 0;
  } else {
    g_poolMisses++;
    b = alloc_record(count);
    if (!b) return nullptr;
  }
  if (data && !upload(b->ptr, data, count)) {
    b->magic = kMagicPooled;
    g_pool[count].push_back(b);
    g_poolBytes += uint64_t(count) * 4;
    return nullptr;
  }
  if (g_capturing) {  // the graph keeps it until ReleaseGraph
    b->refCount++;
    g_captureHeld.push_back(b);
  }
  return b;
}

static void release_internal(Buffer* b) {
  drop_tag(b);
  auto& pool = g_pool[b->count];
  uint64_t bytes = uint64_t(b->count) * 4;
  if (pool.size() < max_pool_for_size(b->count) && g_poolBytes + bytes <= g_poolCapBytes) {
    b->magic = kMagicPooled;
    pool.push_back(b);
    g_poolBytes += bytes;
  } else {
    free_record(b);
  }
}

static void park_buffer(Buffer* b) {
  if (--b->refCount > 0) return;
  if (g_capturing) {
    b->refCount = 1;
    g_captureHeld.push_back(b);
    return;
  }
  drop_tag(b, true);
  b->magic = kMagicPooled;
  g_pool[b->count].push_back(b);
  g_poolBytes += uint64_t(b->count) * 4;
}

void release_buffer(void* h) {
  if (!h) return;
  Buffer* b = static_cast<Buffer*>(h);
  if (b->magic != kMagicLive) {
    set_error("ReleaseBuffer: handle %p is not live (double release?)", h);
    return;
  }
  if (--b->refCount > 0) return;
  if (g_capturing) {  // a recorded node may still read it: the graph keeps it
    b->refCount = 1;
    g_captureHeld.push_back(b);
    return;
  }
  release_internal(b);
}

float* workspace(size_t floats) {
  if (floats <= g_wsFloats) return g_ws;
  size_t want = std::max(floats, g_wsFloats * 3 / 2);
  want = (want + 65535) & ~size_t(65535);
  if (g_ws) {
    if (g_capturing || g_liveGraphs > 0) {
      g_wsRetired.push_back(g_ws);  // a graph may reference it
    } else {
      hipStreamSynchronize(g_stream);
      hipFree(g_ws);
    }
    g_ws = nullptr;
    g_wsFloats = 0;
  }
  if (hipMalloc((void**)&g_ws, want * 4) != hipSuccess) {
    hipGetLastError();
    drain_pool_locked();
    if (hipMalloc((void**)&g_ws, want * 4) != hipSuccess) {
      hipGetLastError();
      g_ws = nullptr;
      set_error("workspace: cannot allocate %zu floats", want);
      return nullptr;
    }
  }
  g_wsFloats = want;
  return g_ws;
}

static void read_pci_device_id(int dev, uint32_t* out) {
  char bus[64] = {0};
  *out = 0;
  if (hipDeviceGetPCIBusId(bus, sizeof(bus), dev) != hipSuccess) return;
  for (char* c = bus; *c; ++c) *c = (char)tolower(*c);
  char path[160];
  snprintf(path, sizeof(path), "/sys/bus/pci/devices/%s/device", bus);
  FILE* f = fopen(path, "r");
  if (!f) return;
  unsigned v = 0;
  if (fscanf(f, "%x", &v) == 1) *out = v;
  fclose(f);
}

}  // namespace dce

using namespace dce;

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

bool InitEngine(void) {
  if (g_init) return true;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    hipGetLastError();
    set_error("InitEngine: no HIP device visible");
    return false;
  }
  const char* env = getenv("DCE_DEVICE");
  g_device = env ? atoi(env) : 0;
  if (g_device < 0 || g_device >= n) g_device = 0;
  if (hipSetDevice(g_device) != hipSuccess) {
    set_error("InitEngine: hipSetDevice(%d) failed", g_device);
    return false;
  }
  // Default priority, non-blocking with respect to the legacy null stream.
  if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
    set_error("InitEngine: stream creation failed");
    return false;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, g_device) != hipSuccess) {
    set_error("InitEngine: hipGetDeviceProperties failed");
    return false;
  }
  g_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  memset(&g_info, 0, sizeof(g_info));
  g_info.vendorId = 0x1002;
  read_pci_device_id(g_device, &g_info.deviceId);
  g_info.dedicatedVRAM = prop.totalGlobalMem;
  g_info.sharedMemory = 0;
  g_info.isIntegrated = prop.integrated ? 1u : 0u;
  snprintf(g_info.description, sizeof(g_info.description), "%s (%s)",
           prop.name[0] ? prop.name : "AMD Instinct GPU", prop.gcnArchName);
  g_poolCapBytes = uint64_t(prop.totalGlobalMem) / 2;
  const float ones[4] = {1.f, 1.f, 1.f, 1.f};
  if (hipMalloc((void**)&g_misc, 1024 * 4) != hipSuccess ||
      hipMalloc((void**)&g_ones, sizeof(ones)) != hipSuccess ||
      hipMemcpy(g_ones, ones, sizeof(ones), hipMemcpyHostToDevice) != hipSuccess) {
    hipGetLastError();
    set_error("InitEngine: scratch allocation failed");
    return false;
  }
  if (!noalloc_setup(g_device)) return false;
  g_init = true;
  g_err[0] = 0;
  return true;
}

void GetGPUInfo(GPUInfo* info) {
  if (!info) return;
  if (!g_init) {
    memset(info, 0, sizeof(*info));
    return;
  }
  *info = g_info;
}

const char* GetLastErrorString(void) { return g_err; }
void ClearLastError(void) { g_err[0] = 0; }

void* CreateBuffer(float* data, uint32_t count) { return create_buffer(data, count); }

void AddRefBuffer(void* handle) {
  if (!handle) return;
  Buffer* b = as_buffer(handle, "AddRefBuffer");
  if (b) b->refCount++;
}

void ReleaseBuffer(void* handle) { release_buffer(handle); }

void ReleaseBufferBatch(void** handles, uint32_t count) {
  if (!handles) return;
  for (uint32_t i = 0; i < count; ++i) release_buffer(handles[i]);
}

void UpdateBuffer(void* handle, float* data) {
  if (!handle || !data || !g_init) return;
  Buffer* b = as_buffer(handle, "UpdateBuffer");
  if (!b) return;
  drop_tag(b);  // the contents are the caller's now
  upload(b->ptr, data, b->count);
}

void ReadBuffer(void* handle, float* dst) {
  if (!handle || !dst || !g_init) return;
  if (refuse_in_capture("ReadBuffer")) return;
  Buffer* b = as_buffer(handle, "ReadBuffer");
  if (!b) return;
  if (hipMemcpyAsync(dst, b->ptr, size_t(b->count) * 4, hipMemcpyDeviceToHost, g_stream) !=
      hipSuccess) {
    set_error("ReadBuffer: copy failed");
  }
  if (hipStreamSynchronize(g_stream) != hipSuccess) set_error("ReadBuffer: stream error");
}

void ClearBuffer(void* handle) {
  if (!handle || !g_init) return;
  Buffer* b = as_buffer(handle, "ClearBuffer");
  if (!b) return;
  drop_tag(b);
  fill_zero(b->ptr, b->count);
}

void FlushGPU(void) {}

void SyncGPU(void) {
  if (g_init && !refuse_in_capture("SyncGPU")) hipStreamSynchronize(g_stream);
}

void WarmPool(uint32_t* sizes, uint32_t numSizes, uint32_t copies) {
  if (!g_init || !sizes || refuse_in_capture("WarmPool")) return;
  for (uint32_t i = 0; i < numSizes; ++i) {
    const uint32_t count = sizes[i];
    if (!count) continue;
    const size_t target = std::min<size_t>(copies, max_pool_for_size(count));
    size_t have = g_pool[count].size();
    for (; have < target; ++have) {
      Buffer* b = alloc_record(count);  // fresh allocations: not pool hits or misses
      if (!b) break;
      release_internal(b);
      if (g_pool[count].size() <= have) break;  // pool byte cap reached (b was freed)
    }
  }
}

void GetPoolStats(uint64_t* hits, uint64_t* misses) {
  if (hits) *hits = g_poolHits;
  if (misses) *misses = g_poolMisses;
}

void ResetPoolStats(void) {
  g_poolHits = 0;
  g_poolMisses = 0;
}

uint64_t GetPoolMemory(void) { return g_poolBytes; }

void DrainPool(void) {
  if (g_init) drain_pool_locked();
}

// ------------------------------------------------------------------ dispatch
bool CompileShader(const char* name, const wchar_t* path) {
  (void)path;
  return name && find_shader(name) != nullptr;
}

bool CompileShaderEx(const char* name, const wchar_t* path, const char* entry) {
  (void)path;
  (void)entry;
  set_error("CompileShaderEx(%s): custom HLSL shaders are not supported", name ? name : "?");
  return false;
}

// A kernel's outputs lose any producer tag (pooling geometry, conv input
// copy) before it runs: their contents are then the kernel's, not the
// producer's that the tag describes.
static void run_entry(const ShaderEntry* e, const Dispatch& d) {
  for (uint32_t i = 0; d.uavs && i < d.nU; ++i) {
    Buffer* b = static_cast<Buffer*>(d.uavs[i]);
    if (b && b->magic == kMagicLive) drop_tag(b);
  }
  e->fn(d);
}

void RunShader(const char* name, void** srvs, uint32_t srvCount, void** uavs,
               uint32_t uavCount, uint32_t* threads, void* cb, uint32_t cbSize) {
  if (!g_init || !name) return;
  const ShaderEntry* e = find_shader(name);
  if (!e) {
    set_error("RunShader: unknown kernel '%s'", name);
    return;
  }
  Dispatch d{srvs, srvCount, uavs, uavCount, threads, static_cast<const uint8_t*>(cb),
             cb ? cbSize : 0u};
  run_entry(e, d);
}

void RunShaderRaw(const char* name, void** srvs, uint32_t srvCount, void** uavs,
                  uint32_t uavCount, uint32_t* threads, void* cb, uint32_t cbSize) {
  RunShader(name, srvs, srvCount, uavs, uavCount, threads, cb, cbSize);
}

void* RunShaderAlloc(const char* name, void** srvs, uint32_t srvCount, uint32_t outCount,
                     uint32_t* threads, void* cb, uint32_t cbSize) {
  void* out = CreateBuffer(nullptr, outCount);
  if (!out) return nullptr;
  void* uavs[1] = {out};
  RunShader(name, srvs, srvCount, uavs, 1, threads, cb, cbSize);
  return out;
}

void* RunShaderAlloc2(const char* name, void** srvs, uint32_t srvCount, uint32_t outCount,
                      void* extraUav, uint32_t* threads, void* cb, uint32_t cbSize) {
  void* out = CreateBuffer(nullptr, outCount);
  if (!out) return nullptr;
  void* uavs[2] = {out, extraUav};
  RunShader(name, srvs, srvCount, uavs, 2, threads, cb, cbSize);
  return out;
}

void* ResolveShader(const char* name) {
  if (!name) return nullptr;
  return const_cast<ShaderEntry*>(find_shader(name));
}

void RunSequence(SeqCmd* cmds, uint32_t count) {
  if (!g_init || !cmds) return;
  for (uint32_t i = 0; i < count; ++i) {
    SeqCmd& c = cmds[i];
    if (!c.shader) continue;
    const ShaderEntry* e = shader_entry(c.shader);
    if (!e) {
      set_error("RunSequence: command %u has an unresolved shader pointer", i);
      continue;
    }
    Dispatch d{c.srvs, std::min<uint32_t>(c.srvCount, 8), c.uavs,
               std::min<uint32_t>(c.uavCount, 4), c.threads, c.cbData,
               std::min<uint32_t>(c.cbSize, 64)};
    run_entry(e, d);
  }
}

void RunSequenceWithSGD(SeqCmd* cmds, uint32_t cmdCount, void** params, void** grads,
                        uint32_t* sizes, uint32_t numParams, float lr, float clip) {
  RunSequence(cmds, cmdCount);
  SGDBatch(params, grads, sizes, numParams, lr, clip);
}

// -------------------------------------------------------------- fused: GEMM
void* MatMulAlloc(void* a, void* b, uint32_t M, uint32_t K, uint32_t N, uint32_t flags) {
  if (!g_init) return nullptr;
  Buffer* A = as_buffer(a, "MatMulAlloc(A)");
  Buffer* B = as_buffer(b, "MatMulAlloc(B)");
  if (!A || !B) return nullptr;
  if (uint64_t(M) * N == 0 || uint64_t(M) * N > 0xFFFFFFFFull) {
    set_error("MatMulAlloc: bad output size %ux%u", M, N);
    return nullptr;
  }
  if (uint64_t(A->count) < uint64_t(M) * K || uint64_t(B->count) < uint64_t(K) * N) {
    set_error("MatMulAlloc: operand smaller than M=%u K=%u N=%u implies", M, K, N);
    return nullptr;
  }
  void* out = create_buffer(nullptr, M * N);
  if (!out) return nullptr;
  if (!gemm(A->ptr, B->ptr, static_cast<Buffer*>(out)->ptr, M, K, N, flags & 3u)) {
    release_buffer(out);
    return nullptr;
  }
  return out;
}

// -------------------------------------------------------------- fused: conv
static bool conv_geom(const char* what, uint32_t B, uint32_t C, uint32_t H, uint32_t W,
                      uint32_t OC, uint32_t kH, uint32_t kW, uint32_t s, uint32_t p,
                      ConvGeom* g) {
  if (kH != kW) {
    set_error("%s: only square kernels are supported (kH=%u kW=%u)", what, kH, kW);
    return false;
  }
  if (!B || !C || !H || !W || !OC || !kH || !s || H + 2 * p < kH || W + 2 * p < kW) {
    set_error("%s: invalid geometry", what);
    return false;
  }
  g->B = B; g->C = C; g->H = H; g->W = W; g->OC = OC; g->k = kH; g->s = s; g->p = p;
  g->OH = (H + 2 * p - kH) / s + 1;
  g->OW = (W + 2 * p - kW) / s + 1;
  uint64_t xs = uint64_t(B) * C * H * W, ys = uint64_t(B) * OC * g->OH * g->OW;
  // The filters too: the callers' 32-bit buffer-size checks rely on it.
  uint64_t ws = uint64_t(OC) * C * kH * kW;
  if (xs >= (1ull << 31) || ys >= (1ull << 31) || ws >= (1ull << 31)) {
    set_error("%s: tensor too large for 31-bit indexing", what);
    return false;
  }
  return true;
}

void* ConvForwardFused(void* x, void* filters, void* bias, uint32_t batch, uint32_t inC,
                       uint32_t inH, uint32_t inW, uint32_t outC, uint32_t kH, uint32_t kW,
                       uint32_t stride, uint32_t padding, uint32_t actType, void** pIm2col) {
  if (pIm2col) *pIm2col = nullptr;
  if (!g_init) return nullptr;
  ConvGeom g;
  if (!conv_geom("ConvForwardFused", batch, inC, inH, inW, outC, kH, kW, stride, padding, &g))
    return nullptr;
  Buffer* X = as_buffer(x, "ConvForwardFused(x)");
  Buffer* Wt = as_buffer(filters, "ConvForwardFused(filters)");
  Buffer* Bi = as_buffer(bias, "ConvForwardFused(bias)");
  if (!X || !Wt || !Bi) return nullptr;
  if (X->count < batch * inC * inH * inW || Wt->count < outC * inC * kH * kW ||
      Bi->count < outC) {
    set_error("ConvForwardFused: buffer smaller than geometry");
    return nullptr;
  }
  void* out = create_buffer(nullptr, batch * outC * g.OH * g.OW);
  if (!out) return nullptr;
  // The "im2col" handle of this backend is the channel-innermost copy of x
  // that the forward builds anyway; ConvBackwardFused reuses and releases it.
  void* keep = nullptr;
  if (pIm2col) {
    keep = create_buffer(nullptr, uint32_t(xcopy_floats(g)));
    if (!keep) {
      release_buffer(out);
      return nullptr;
    }
  }
  Buffer* K = static_cast<Buffer*>(keep);
  // With no activation a batch norm usually follows: the GEMM leaves the
  // statistics of y in a side buffer, which batchnorm_mean_var on y reads
  // instead of making its own pass over y.
  struct StatsCtx {
    Buffer* side;
    uint32_t C;
  } sctx{nullptr, outC};
  ConvStatsReq sreq{[](void* ctx, uint32_t pieces) -> double* {
                      StatsCtx* c = static_cast<StatsCtx*>(ctx);
                      const uint64_t n = uint64_t(c->C) * pieces * 4;  // two doubles per piece
                      if (n >= 0xFFFFFFFFull) return nullptr;
                      c->side = static_cast<Buffer*>(create_buffer(nullptr, uint32_t(n)));
                      return c->side ? reinterpret_cast<double*>(c->side->ptr) : nullptr;
                    },
                    &sctx, 0};
  if (!conv_forward(X->ptr, K ? K->ptr : nullptr, Wt->ptr, Bi->ptr,
                    static_cast<Buffer*>(out)->ptr, g, actType, actType == 0 ? &sreq : nullptr)) {
    release_buffer(out);
    release_buffer(keep);
    release_buffer(sctx.side);
    return nullptr;
  }
  if (sctx.side) {
    if (sreq.pieces) {
      const bool gn = conv_g_nhwc_pass(g);
      tag_bn_stats(out, sctx.side, batch, outC, g.OH * g.OW, sreq.pieces, gn ? g.OH : 0,
                   gn ? g.OW : 0);
    }
    else
      release_buffer(sctx.side);
  }
  if (K) {
    K->tag = kNhwcTag;
    K->meta[0] = batch;
    K->meta[1] = inC;
    K->meta[2] = inH;
    K->meta[3] = inW;
    K->meta[4] = xcopy_tag(g);
    *pIm2col = keep;
  }
  if (actType == 1 && conv_g_layout(g) == kGLayoutPad) {
    // A max-pool over this output can then make its backward's masked G.
    Buffer* Y = static_cast<Buffer*>(out);
    set_tag(Y, kReluOutTag);
    Y->meta[0] = conv_g_layout(g);
    Y->meta[1] = batch;
    Y->meta[2] = outC;
    Y->meta[3] = g.OH;
    Y->meta[4] = g.OW;
  }
  return out;
}

void ConvBackwardFused(void* gradOut, void* fwdOut, void* x, void* filters, void* im2col,
                       uint32_t batch, uint32_t inC, uint32_t inH, uint32_t inW,
                       uint32_t outC, uint32_t kH, uint32_t kW, uint32_t stride,
                       uint32_t padding, uint32_t actType, uint32_t xReq, uint32_t wReq,
                       uint32_t bReq, void** pDFilters, void** pDBias, void** pDInput) {
  if (pDFilters) *pDFilters = nullptr;
  if (pDBias) *pDBias = nullptr;
  if (pDInput) *pDInput = nullptr;
  if (!g_init) return;
  ConvGeom g;
  bool ok = conv_geom("ConvBackwardFused", batch, inC, inH, inW, outC, kH, kW, stride,
                      padding, &g);
  Buffer* DY = ok ? as_buffer(gradOut, "ConvBackwardFused(grad)") : nullptr;
  Buffer* X = DY ? as_buffer(x, "ConvBackwardFused(x)") : nullptr;
  Buffer* Wt = X ? as_buffer(filters, "ConvBackwardFused(filters)") : nullptr;
  Buffer* Y = nullptr;
  if (Wt && actType == 1 && fwdOut) Y = as_buffer(fwdOut, "ConvBackwardFused(fwd_output)");
  uint32_t ysz = batch * outC * g.OH * g.OW;
  if (Wt && (actType != 1 || !fwdOut || Y)) {
    if (DY->count < ysz || (Y && Y->count < ysz) || X->count < batch * inC * inH * inW ||
        Wt->count < outC * inC * kH * kW) {
      set_error("ConvBackwardFused: buffer smaller than geometry");
    } else {
      const float* yp = Y ? Y->ptr : nullptr;
      // dy from MaxPoolBackwardFused over this very output (unchanged since):
      // its masked G is already made.
      PreG pre{};
      const PreG* pp = nullptr;
      const bool gMatch = DY->tag == kGradGTag && DY->side && DY->meta[1] == batch &&
                          DY->meta[2] == outC && DY->meta[3] == g.OH && DY->meta[4] == g.OW;
      // A ReLU conv's masked G (the max-pool backward over its output), or
      // the plain NHWC G of dy (the batch-norm backward that made dy) for a
      // conv with no ReLU mask.
      if ((Y && gMatch && DY->src == Y && tag_alive(Y, kReluOutTag, DY->srcGen) &&
           DY->meta[0] == conv_g_layout(g)) ||
          (!Y && actType != 1 && gMatch && DY->meta[0] == kGLayoutNhwc && conv_g_nhwc_pass(g))) {
        pre.layout = DY->meta[0];
        pre.g = DY->side->ptr;
        pre.db = pre.g + g_side_floats(pre.layout, batch, outC, g.OH, g.OW);
        pre.dbRows = DY->aux32;
        pp = &pre;
      }
      const float* xn = nullptr;
      if (im2col) {
        Buffer* Kb = static_cast<Buffer*>(im2col);
        if (Kb->magic == kMagicLive && Kb->tag == kNhwcTag && Kb->meta[0] == batch &&
            Kb->meta[1] == inC && Kb->meta[2] == inH && Kb->meta[3] == inW &&
            Kb->meta[4] == xcopy_tag(g) && Kb->count >= xcopy_floats(g))
          xn = Kb->ptr;
      }
      bool wantW = wReq && pDFilters, wantB = bReq && pDBias, wantX = xReq && pDInput;
      void* dW = wantW ? create_buffer(nullptr, outC * inC * kH * kW) : nullptr;
      void* dB = wantB ? create_buffer(nullptr, outC) : nullptr;
      void* dX = wantX ? create_buffer(nullptr, batch * inC * inH * inW) : nullptr;
      bool good = (!wantW || dW) && (!wantB || dB) && (!wantX || dX);
      if (good && (wantW || wantB || wantX))
        good = conv_backward(DY->ptr, yp, X->ptr, xn, Wt->ptr,
                             dW ? static_cast<Buffer*>(dW)->ptr : nullptr,
                             dB ? static_cast<Buffer*>(dB)->ptr : nullptr,
                             dX ? static_cast<Buffer*>(dX)->ptr : nullptr, g, pp);
      if (good) {
        if (pDFilters) *pDFilters = dW;
        if (pDBias) *pDBias = dB;
        if (pDInput) *pDInput = dX;
      } else {
        release_buffer(dW);
        release_buffer(dB);
        release_buffer(dX);
      }
    }
  }
  // The reference releases the im2col handle it is given (engine.cpp:877).
  if (im2col) release_buffer(im2col);
}

// ----------------------------------------------------------- fused: maxpool
void* MaxPoolForwardFused(void* x, uint32_t batch, uint32_t inC, uint32_t inH, uint32_t inW,
                          uint32_t poolSize, uint32_t stride, void** pIndices) {
  if (pIndices) *pIndices = nullptr;
  if (!g_init) return nullptr;
  Buffer* X = as_buffer(x, "MaxPoolForwardFused(x)");
  if (!X) return nullptr;
  if (!poolSize || !stride || inH < poolSize || inW < poolSize || !batch || !inC) {
    set_error("MaxPoolForwardFused: invalid geometry");
    return nullptr;
  }
  if (uint64_t(batch) * inC * inH * inW >= (1ull << 31) ||
      X->count < batch * inC * inH * inW) {
    set_error("MaxPoolForwardFused: input buffer does not match geometry");
    return nullptr;
  }
  uint32_t OH = (inH - poolSize) / stride + 1, OW = (inW - poolSize) / stride + 1;
  uint32_t n = batch * inC * OH * OW;
  void* out = create_buffer(nullptr, n);
  void* idx = create_buffer(nullptr, n);
  if (!out || !idx) {
    release_buffer(out);
    release_buffer(idx);
    return nullptr;
  }
  Buffer* I = static_cast<Buffer*>(idx);
  if (!maxpool_forward(X->ptr, static_cast<Buffer*>(out)->ptr, I->ptr, batch, inC, inH, inW,
                       poolSize, stride, OH, OW)) {
    release_buffer(out);
    release_buffer(idx);
    return nullptr;
  }
  set_tag(I, kPoolTag);
  I->meta[0] = inH;
  I->meta[1] = inW;
  I->meta[2] = poolSize;
  I->meta[3] = stride;
  // Links for the masked backward: the pooled values, and the input when it
  // is a ReLU conv output of this geometry.
  Buffer* P = static_cast<Buffer*>(out);
  set_tag(P, kPoolOutTag);
  I->aux = P;
  I->auxGen = P->gen;
  if (X->tag == kReluOutTag && X->meta[1] == batch && X->meta[2] == inC && X->meta[3] == inH &&
      X->meta[4] == inW) {
    I->src = X;
    I->srcGen = X->gen;
  }
  if (pIndices)
    *pIndices = idx;
  else
    release_buffer(idx);
  return out;
}

void* MaxPoolBackwardFused(void* gradOut, void* indices, uint32_t batch, uint32_t inC,
                           uint32_t outH, uint32_t outW, uint32_t xSize) {
  if (!g_init) return nullptr;
  Buffer* DZ = as_buffer(gradOut, "MaxPoolBackwardFused(grad)");
  Buffer* I = DZ ? as_buffer(indices, "MaxPoolBackwardFused(indices)") : nullptr;
  void* dx = nullptr;
  const uint64_t n64 = uint64_t(batch) * inC * outH * outW;
  const uint32_t n = uint32_t(n64);
  if (I && n64 >= (1ull << 31)) {
    set_error("MaxPoolBackwardFused: tensor too large for 31-bit indexing");
  } else if (I && (DZ->count < n || I->count < n)) {
    set_error("MaxPoolBackwardFused: buffer smaller than geometry");
  } else if (I) {
    dx = create_buffer(nullptr, xSize);
    if (dx) {
      uint32_t H = 0, W = 0, k = 0, s = 0;
      const uint32_t* m = I->meta;
      if (I->tag == kPoolTag && uint64_t(batch) * inC * m[0] * m[1] == xSize &&
          (m[0] - m[2]) / m[3] + 1 == outH && (m[1] - m[2]) / m[3] + 1 == outW) {
        H = m[0]; W = m[1]; k = m[2]; s = m[3];
      }
      // Over a ReLU conv output (unchanged since the forward, as are the
      // pooled values): also the conv backward's masked G, owned by dx.
      Buffer* DX = static_cast<Buffer*>(dx);
      Buffer* X = H ? I->src : nullptr;
      const uint32_t lay = X ? X->meta[0] : 0;
      Buffer* side = nullptr;
      if (X && tag_alive(X, kReluOutTag, I->srcGen) && tag_alive(I->aux, kPoolOutTag, I->auxGen) &&
          I->aux->count >= n && maxpool_backward_g_ok(inC, H, W, outH, outW, k, s, lay)) {
        const size_t nG = g_side_floats(lay, batch, inC, H, W);
        const uint32_t rows = maxpool_backward_g_rows(batch, H, W, lay);
        const size_t total = nG + size_t(rows) * inC;
        if (total < 0xFFFFFFFFull) side = static_cast<Buffer*>(create_buffer(nullptr, uint32_t(total)));
        if (side) {
          if (maxpool_backward_g(DZ->ptr, I->ptr, I->aux->ptr, DX->ptr, side->ptr, side->ptr + nG,
                                 batch, inC, outH, outW, H, W, k, lay, (W + 3u) & ~3u)) {
            set_tag(DX, kGradGTag);
            DX->side = side;
            DX->src = X;
            DX->srcGen = X->gen;
            DX->meta[0] = lay;
            DX->meta[1] = batch;
            DX->meta[2] = inC;
            DX->meta[3] = H;
            DX->meta[4] = W;
            DX->aux32 = rows;
          } else {
            release_buffer(side);
            release_buffer(dx);
            dx = nullptr;
          }
        }
      }
      if (dx && !side &&
          !maxpool_backward(DZ->ptr, I->ptr, DX->ptr, batch, inC, outH, outW, xSize, H, W, k, s)) {
        release_buffer(dx);
        dx = nullptr;
      }
    }
  }
  // The reference releases the indices after routing (engine.cpp:928).
  if (indices) release_buffer(indices);
  return dx;
}

// ---------------------------------------------------------------- optimisers
void SGDBatch(void** params, void** grads, uint32_t* sizes, uint32_t numParams, float lr,
              float clip) {
  if (!g_init || !params || !grads || !sizes || !numParams) return;
  drop_tags(params, numParams);
  sgd_multi(params, grads, sizes, numParams, lr, clip);
}

float SGDBatchClipped(void** params, void** grads, uint32_t* sizes, uint32_t numParams,
                      float lr, float maxNorm) {
  if (!g_init || !params || !grads || !sizes || !numParams) return 0.0f;
  drop_tags(params, numParams);
  float* d_ns = g_misc;  // [norm, scale]
  if (!grad_norm_multi(grads, sizes, numParams, maxNorm, d_ns)) return 0.0f;
  if (!sgd_scaled_multi(params, grads, sizes, numParams, lr, d_ns)) return 0.0f;
  if (g_capturing) return std::nanf("");  // the norm is known only when the graph runs
  float h[2] = {0, 0};
  hipMemcpyAsync(h, d_ns, 8, hipMemcpyDeviceToHost, g_stream);
  hipStreamSynchronize(g_stream);
  return h[0];
}

void AdamBatch(void** params, void** grads, void** m, void** v, uint32_t* sizes,
               uint32_t numParams, float stepSize, float beta1, float beta2, float eps,
               float weightDecay, float clip) {
  if (!g_init || !params || !grads || !m || !v || !sizes || !numParams) return;
  drop_tags(params, numParams);
  drop_tags(m, numParams);
  drop_tags(v, numParams);
  adam_multi(params, grads, m, v, sizes, numParams, stepSize, beta1, beta2, eps, weightDecay,
             clip);
}

float ClipGradNorm(void** grads, uint32_t* sizes, uint32_t numGrads, float maxNorm) {
  if (!g_init || !grads || !sizes || !numGrads) return 0.0f;
  drop_tags(grads, numGrads);
  float* ns = g_misc;  // [norm, scale]
  if (!grad_norm_multi(grads, sizes, numGrads, maxNorm, ns)) return 0.0f;
  if (!scale_grads_multi(grads, sizes, numGrads, ns)) return 0.0f;
  if (g_capturing) return std::nanf("");  // the norm is known only when the graph runs
  float h[2] = {0, 0};
  hipMemcpyAsync(h, ns, 8, hipMemcpyDeviceToHost, g_stream);
  hipStreamSynchronize(g_stream);
  return h[0];
}

void AdamBatchCounted(void** params, void** grads, void** m, void** v, uint32_t* sizes,
                      uint32_t numParams, void* stepState, uint32_t t, float stepSize, double lr,
                      double beta1, double beta2, float eps, float weightDecay, float clip) {
  if (!g_init || !params || !grads || !m || !v || !sizes || !numParams) return;
  drop_tags(params, numParams);
  drop_tags(m, numParams);
  drop_tags(v, numParams);
  Buffer* st = as_buffer(stepState, "AdamBatchCounted(stepState)");
  if (!st) return;
  if (st->count < 2) {
    set_error("AdamBatchCounted: the step state buffer needs 2 floats (has %u)", st->count);
    return;
  }
  adam_counted_multi(params, grads, m, v, sizes, numParams, st->ptr, t, stepSize, lr, beta1,
                     beta2, eps, weightDecay, clip);
}

float ClipGradNormNoAlloc(void** grads, uint32_t* sizes, uint32_t numGrads, float maxNorm) {
  if (!g_init) {
    set_error("ClipGradNormNoAlloc: engine not initialised");
    return -1.0f;
  }
  if (!grads || !sizes || !numGrads) return 0.0f;
  drop_tags(grads, numGrads, true);
  return clip_grad_norm_noalloc(g_device, grads, sizes, numGrads, maxNorm, g_capturing);
}

// ----------------------------------------------------------------- profiling
void SetProfiling(int enabled) {
  if (!enabled) resolve_profile();
  g_prof = enabled != 0;
}

bool GetProfile(const char* family, uint64_t* launches, double* ms, double* flops,
                double* bytes) {
  resolve_profile();
  if (!family) return false;
  auto it = g_profStats.find(family);
  if (it == g_profStats.end()) return false;
  if (launches) *launches = it->second.launches;
  if (ms) *ms = it->second.ms;
  if (flops) *flops = it->second.flops;
  if (bytes) *bytes = it->second.bytes;
  return true;
}

void ResetProfile(void) {
  resolve_profile();
  g_profStats.clear();
}

// ------------------------------------------------------------ graph capture
struct GraphRec {
  uint32_t magic;
  hipGraphExec_t exec;
  std::vector<Buffer*> held;
};
constexpr uint32_t kMagicGraph = 0xDC6A9A7Fu;

static void abort_capture() {
  g_capturing = false;
  std::vector<Buffer*> held;
  held.swap(g_captureHeld);
  for (Buffer* b : held) release_buffer(b);
}

bool BeginCapture(void) {
  if (!ensure_init()) return false;
  if (g_capturing) {
    set_error("BeginCapture: a capture is already open");
    return false;
  }
  resolve_profile();
  if (hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
    hipGetLastError();
    set_error("BeginCapture: hipStreamBeginCapture failed");
    return false;
  }
  g_capturing = true;
  g_captureFailed = false;
  g_captureHeld.clear();
  return true;
}

void* EndCapture(void) {
  if (!g_capturing) {
    set_error("EndCapture: no capture is open");
    return nullptr;
  }
  hipGraph_t graph = nullptr;
  const hipError_t e = hipStreamEndCapture(g_stream, &graph);
  if (e != hipSuccess || g_captureFailed || !graph) {
    if (e != hipSuccess) hipGetLastError();
    if (graph) hipGraphDestroy(graph);
    const bool failed = g_captureFailed;
    abort_capture();
    if (!failed) set_error("EndCapture: hipStreamEndCapture failed");
    return nullptr;
  }
  hipGraphExec_t exec = nullptr;
  if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
    hipGetLastError();
    hipGraphDestroy(graph);
    abort_capture();
    set_error("EndCapture: hipGraphInstantiate failed");
    return nullptr;
  }
  hipGraphDestroy(graph);
  GraphRec* g = new GraphRec{kMagicGraph, exec, std::move(g_captureHeld)};
  g_captureHeld.clear();
  g_capturing = false;
  g_liveGraphs++;
  return g;
}

bool ReplayGraph(void* graph) {
  GraphRec* g = static_cast<GraphRec*>(graph);
  if (!g_init || !g || g->magic != kMagicGraph) {
    set_error("ReplayGraph: not a live graph handle");
    return false;
  }
  if (refuse_in_capture("ReplayGraph")) return false;
  if (hipGraphLaunch(g->exec, g_stream) != hipSuccess) {
    hipGetLastError();
    set_error("ReplayGraph: hipGraphLaunch failed");
    return false;
  }
  return true;
}

void ReleaseGraph(void* graph) {
  GraphRec* g = static_cast<GraphRec*>(graph);
  if (!g || g->magic != kMagicGraph) return;
  if (refuse_in_capture("ReleaseGraph")) return;
  hipStreamSynchronize(g_stream);
  hipGraphExecDestroy(g->exec);
  for (Buffer* b : g->held) release_buffer(b);
  g->magic = 0;
  delete g;
  if (--g_liveGraphs == 0) {
    for (float* p : g_wsRetired) hipFree(p);
    g_wsRetired.clear();
  }
}

// One event pair around everything queued between the two calls, recorded as
// one launch of `family` (the name is kept for the process's lifetime).
static hipEvent_t g_regionEv = nullptr;
static const char* g_regionFam = nullptr;
static double g_regionFlops = 0, g_regionBytes = 0;

bool BeginProfileRegion(const char* family, double flops, double bytes) {
  static std::set<std::string> names;
  if (!ensure_init() || !family || g_capturing || g_regionEv) {
    set_error("BeginProfileRegion: not initialised, no family, capturing, or a region is open");
    return false;
  }
  g_regionFam = names.insert(family).first->c_str();
  g_regionFlops = flops;
  g_regionBytes = bytes;
  g_regionEv = take_event();
  if (!g_regionEv) return false;
  hipEventRecord(g_regionEv, g_stream);
  return true;
}

bool EndProfileRegion(void) {
  if (!g_regionEv) {
    set_error("EndProfileRegion: no region is open");
    return false;
  }
  hipEvent_t e1 = take_event();
  if (!e1) return false;
  hipEventRecord(e1, g_stream);
  g_profPending.push_back({g_regionFam, g_regionEv, e1, g_regionFlops, g_regionBytes});
  g_regionEv = nullptr;
  return true;
}

double SetStreamingThreshold(double bytes) {
  const double prev = g_streamBytes;
  g_streamBytes = bytes < 0 ? kStreamBytes : bytes;
  return prev;
}

void SetProfileFilter(const char* families) {
  resolve_profile();
  g_profFilter.clear();
  if (!families) return;
  std::string cur;
  for (const char* c = families;; ++c) {
    if (*c == ',' || *c == 0) {
      if (!cur.empty()) g_profFilter.push_back(cur);
      cur.clear();
      if (*c == 0) break;
    } else if (*c != ' ') {
      cur.push_back(*c);
    }
  }
}

}  // extern "C"
