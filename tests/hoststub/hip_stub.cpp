// A host-only stand-in for the HIP runtime and for the library's kernel launchers, for CPU tests of the library's
// host code (TEST INFRASTRUCTURE: built by tests/hoststub/build.py into tests/hoststub/_build/, never shipped).
//
// Device memory is host memory; nothing runs on a GPU. The point is the bookkeeping: every allocation is tracked, and
// the stand-in records a violation (read back with hipstub_violations) whenever the library
//   - allocates, frees, sets memory, changes a kernel attribute or waits on a stream while a stream is capturing;
//   - frees memory that a live captured graph (or graph exec) still references;
//   - launches (eagerly or by replaying a graph) a kernel whose arguments point into freed memory;
//   - destroys a graph exec while replays are notionally still running (a replay not followed by a wait).
// The launchers record the device pointers of their argument structs (LinArgs, MoeArgs), so a captured graph knows
// every buffer it will read or write.
#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../ijah_amd/csrc/kernels.h"

namespace {

std::recursive_mutex mu;
struct Alloc {
  size_t n;
  bool live;
};
std::map<uintptr_t, Alloc> allocs;   // base -> size, live
std::vector<std::string> violations;
struct Graph {
  std::set<uintptr_t> uses;  // allocation bases its launches reference
  bool live = true;
};
std::map<uintptr_t, Graph> graphs, execs;
uintptr_t next_handle = 0x1000;
bool capturing = false;
hipStream_t cap_stream = nullptr;
Graph cap;                    // launches recorded by the open capture
int replays_unsynced = 0;     // graph replays since the last wait
int graph_launches = 0;

void violation(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  violations.push_back(buf);
}
// the allocation holding address p (live or freed), or allocs.end()
std::map<uintptr_t, Alloc>::iterator find_alloc(uintptr_t p) {
  auto it = allocs.upper_bound(p);
  if (it == allocs.begin()) return allocs.end();
  --it;
  return p < it->first + std::max<size_t>(it->second.n, 1) ? it : allocs.end();
}
void no_capture(const char *what) {
  if (capturing) violation("%s while a stream is capturing", what);
}
// a kernel argument pointer: must be null or inside a live allocation; recorded into the open capture
void use(const void *ptr, const char *kernel) {
  if (!ptr) return;
  const uintptr_t p = (uintptr_t)ptr;
  auto it = find_alloc(p);
  if (it == allocs.end()) return;  // not device memory the stand-in made (e.g. a host scalar): not tracked
  if (!it->second.live) violation("%s: argument %p points into freed memory", kernel, ptr);
  if (capturing) cap.uses.insert(it->first);
}
void check_graph(const Graph &g, const char *what) {
  for (uintptr_t b : g.uses) {
    auto it = allocs.find(b);
    if (it == allocs.end() || !it->second.live) violation("%s: a captured launch references freed memory %p", what,
                                                          (void *)b);
  }
}

}  // namespace

extern "C" {

// ---- test hooks
int hipstub_violations(char *out, int n) {
  std::lock_guard<std::recursive_mutex> g(mu);
  std::string all;
  for (const std::string &v : violations) all += v + "\n";
  if (out && n > 0) snprintf(out, (size_t)n, "%s", all.c_str());
  return (int)violations.size();
}
void hipstub_reset() {
  std::lock_guard<std::recursive_mutex> g(mu);
  violations.clear();
  graph_launches = 0;
}
int hipstub_graph_launches() { return graph_launches; }
int hipstub_live_graphs() {
  std::lock_guard<std::recursive_mutex> g(mu);
  int n = 0;
  for (auto &e : execs) n += e.second.live;
  for (auto &e : graphs) n += e.second.live;
  return n;
}
int hipstub_capturing() { return capturing ? 1 : 0; }
void *hipstub_library_stream() { return (void *)ijah::stream(); }
// opens / closes a capture on the library's stream around library calls (to check that the library refuses work
// that must not be captured)
int hipstub_begin_capture() { return hipStreamBeginCapture(ijah::stream(), hipStreamCaptureModeThreadLocal); }
int hipstub_end_capture() {
  hipGraph_t g = nullptr;
  const int r = hipStreamEndCapture(ijah::stream(), &g);
  if (g) hipGraphDestroy(g);
  return r;
}

// ---- the runtime
hipError_t hipGetDeviceCount(int *n) {
  *n = 1;
  return hipSuccess;
}
hipError_t hipGetDevice(int *d) {
  *d = 0;
  return hipSuccess;
}
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_tR0600 *p, int) {
  memset(p, 0, sizeof *p);
  snprintf(p->name, sizeof p->name, "host stand-in");
  snprintf(p->gcnArchName, sizeof p->gcnArchName, "none");
  p->multiProcessorCount = 256;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t, int) {
  *v = 256;
  return hipSuccess;
}
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "hipSuccess" : "stand-in error"; }
hipError_t hipGetLastError() { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) {
  std::lock_guard<std::recursive_mutex> g(mu);
  *s = (hipStream_t)(next_handle += 16);
  return hipSuccess;
}
hipError_t hipMalloc(void **p, size_t n) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipMalloc");
  *p = calloc(1, std::max<size_t>(n, 1));  // kept until the process ends, so that freed addresses stay distinct
  allocs[(uintptr_t)*p] = {n, true};
  return hipSuccess;
}
hipError_t hipFree(void *p) {
  std::lock_guard<std::recursive_mutex> g(mu);
  if (!p) return hipSuccess;
  no_capture("hipFree");
  auto it = allocs.find((uintptr_t)p);
  if (it == allocs.end() || !it->second.live) {
    violation("hipFree(%p): not a live allocation", p);
    return hipErrorInvalidValue;
  }
  for (auto &e : execs)
    if (e.second.live && e.second.uses.count((uintptr_t)p)) violation("hipFree(%p): a live graph exec uses it", p);
  if (capturing && cap.uses.count((uintptr_t)p)) violation("hipFree(%p): the open capture uses it", p);
  it->second.live = false;
  return hipSuccess;
}
hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipMemcpy");
  memcpy(d, s, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind, hipStream_t) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipMemcpyAsync");
  memcpy(d, s, n);
  return hipSuccess;
}
hipError_t hipMemset(void *d, int v, size_t n) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipMemset");
  memset(d, v, n);
  return hipSuccess;
}
hipError_t hipMemsetAsync(void *d, int v, size_t n, hipStream_t) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipMemsetAsync");
  memset(d, v, n);
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) {
  std::lock_guard<std::recursive_mutex> g(mu);
  no_capture("hipStreamSynchronize");
  replays_unsynced = 0;
  return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus *st) {
  *st = capturing && s == cap_stream ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
  std::lock_guard<std::recursive_mutex> g(mu);
  if (capturing) {
    violation("hipStreamBeginCapture while a capture is open");
    return hipErrorIllegalState;
  }
  capturing = true;
  cap_stream = s;
  cap = Graph();
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t *g) {
  std::lock_guard<std::recursive_mutex> l(mu);
  if (!capturing || s != cap_stream) {
    violation("hipStreamEndCapture without an open capture on that stream");
    return hipErrorIllegalState;
  }
  capturing = false;
  const uintptr_t h = next_handle += 16;
  graphs[h] = cap;
  *g = (hipGraph_t)h;
  return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t *ge, hipGraph_t g, hipGraphNode_t *, char *, size_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  auto it = graphs.find((uintptr_t)g);
  if (it == graphs.end() || !it->second.live) {
    violation("hipGraphInstantiate of a dead graph");
    return hipErrorInvalidValue;
  }
  const uintptr_t h = next_handle += 16;
  execs[h] = it->second;
  *ge = (hipGraphExec_t)h;
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t ge, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  no_capture("hipGraphLaunch");
  auto it = execs.find((uintptr_t)ge);
  if (it == execs.end() || !it->second.live) {
    violation("hipGraphLaunch of a dead graph exec");
    return hipErrorInvalidValue;
  }
  check_graph(it->second, "hipGraphLaunch");
  replays_unsynced++;
  graph_launches++;
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t ge) {
  std::lock_guard<std::recursive_mutex> l(mu);
  auto it = execs.find((uintptr_t)ge);
  if (it == execs.end() || !it->second.live) {
    violation("hipGraphExecDestroy of a dead graph exec");
    return hipErrorInvalidValue;
  }
  if (replays_unsynced) violation("hipGraphExecDestroy with %d replays not waited for", replays_unsynced);
  it->second.live = false;
  return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) {
  std::lock_guard<std::recursive_mutex> l(mu);
  auto it = graphs.find((uintptr_t)g);
  if (it == graphs.end() || !it->second.live) {
    violation("hipGraphDestroy of a dead graph");
    return hipErrorInvalidValue;
  }
  it->second.live = false;
  return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t *e) {
  std::lock_guard<std::recursive_mutex> l(mu);
  *e = (hipEvent_t)(next_handle += 16);
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  replays_unsynced = 0;
  return hipSuccess;
}
hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) {
  *ms = 1e-3f;
  return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }
hipError_t hipLaunchKernel(const void *, dim3, dim3, void **, size_t, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  violation("hipLaunchKernel: no kernels in the host stand-in");
  return hipErrorInvalidDeviceFunction;
}

}  // extern "C"

// ---- the library's device-side functions (kernel launchers and shape helpers defined in its .hip sources)
namespace ijah {

static void attr(const char *what) {
  std::lock_guard<std::recursive_mutex> l(mu);
  no_capture(what);
}
void init_batch_attrs() { attr("hipFuncSetAttribute (batch kernels)"); }
void init_fused_attrs() { attr("hipFuncSetAttribute (fused step)"); }
void init_lin_attrs() { attr("hipFuncSetAttribute (linears)"); }
const KernelEntry *find_kernel(const char *, const ne_fconst *, int) { return nullptr; }
uint8_t *noalloc_scratch() {
  static void *p = nullptr;
  if (!p) (void)hipMalloc(&p, kNoAllocScratchBytes);
  return (uint8_t *)p;
}
static void use_lin(const LinArgs &a, const char *k) {
  for (const void *p : {(const void *)a.tiles, (const void *)a.suh, (const void *)a.svh, (const void *)a.x,
                        (const void *)a.y, (const void *)a.xh, (const void *)a.part, (const void *)a.cnt,
                        (const void *)a.epi.e0, (const void *)a.epi.e1, (const void *)a.epi.e2, (const void *)a.epi.e3,
                        (const void *)a.epi.e4, (const void *)a.epi.w16, (const void *)a.epi.ctr})
    use(p, k);
}
void launch_lin(const LinArgs &a, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  use_lin(a, "lin");
}
void launch_lin_multi(const LinArgs *a, int n, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  for (int i = 0; i < n; i++) use_lin(a[i], "lin_multi");
}
void launch_zero_u32(uint32_t *p, size_t, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  use(p, "zero_u32");
}
void launch_decode(const uint32_t *t, int, int, int, uint16_t *w, hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  use(t, "decode");
  use(w, "decode");
}
void launch_hc_prep(const float *h, const uint16_t *nw, const uint16_t *iw, float *xn, float *ip, float *inj, int, int,
                    hipStream_t) {
  std::lock_guard<std::recursive_mutex> l(mu);
  for (const void *p : {(const void *)h, (const void *)nw, (const void *)iw, (const void *)xn, (const void *)ip,
                        (const void *)inj})
    use(p, "hc_prep");
}
void launch_fill_u32(uint32_t *p, uint64_t, uint64_t, hipStream_t) { use(p, "fill"); }
void launch_fill_scale_f16(uint16_t *p, uint64_t, uint64_t, hipStream_t) { use(p, "fill"); }
void launch_fill_normal_bf16(uint16_t *p, uint64_t, uint64_t, float, hipStream_t) { use(p, "fill"); }
void launch_fill_q8_sb(uint32_t *p, uint64_t, int, uint64_t, hipStream_t) { use(p, "fill"); }
// the MoE layer is not exercised by the stand-in: its launchers only check their pointers
static void use_moe(const MoeArgs &a, const char *k) {
  std::lock_guard<std::recursive_mutex> l(mu);
  for (const void *p : {(const void *)a.x, (const void *)a.y, (const void *)a.router, (const void *)a.experts,
                        (const void *)a.shared, (const void *)a.logits, (const void *)a.route, (const void *)a.sgv,
                        (const void *)a.guo, (const void *)a.dn, (const void *)a.sync, (const void *)a.units,
                        (const void *)a.part, (const void *)a.fsync, (const void *)a.q8, (const void *)a.q8gu,
                        (const void *)a.q8o})
    use(p, k);
}
void launch_moe_router(const MoeArgs &a, hipStream_t) { use_moe(a, "moe_router"); }
void launch_moe_gateup(const MoeArgs &a, hipStream_t) { use_moe(a, "moe_gateup"); }
void launch_moe_down(const MoeArgs &a, hipStream_t) { use_moe(a, "moe_down"); }
void launch_moe_combine(const MoeArgs &a, hipStream_t) { use_moe(a, "moe_combine"); }
void launch_moe_fused(const MoeArgs &a, int, hipStream_t) { use_moe(a, "moe_fused"); }
void launch_moe_q8(const MoeArgs &a, hipStream_t) { use_moe(a, "moe_q8"); }
void launch_q8_bf16(const uint8_t *q, uint16_t *b, int, int, hipStream_t) {
  use(q, "q8_bf16");
  use(b, "q8_bf16");
}
void launch_moe_batch(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t) {
  use_moe(a, "moe_batch");
  std::lock_guard<std::recursive_mutex> l(mu);
  for (const void *p : {(const void *)b.bk, (const void *)b.chunks, (const void *)b.rows, (const void *)b.xh,
                        (const void *)b.hh, (const void *)b.dnw, (const void *)b.vpart, (const void *)b.vep})
    use(p, "moe_batch");
}
ExpertLayout expert_layout(int hid, int inter, int K) {  // the same regions, packed (no alignment padding needed)
  ExpertLayout L;
  L.K = K;
  const uint64_t t = (uint64_t)hid * inter * K / 8;
  L.tr[0] = 0, L.tr[1] = t, L.tr[2] = 2 * t;
  L.su[0] = 3 * t, L.sv[0] = L.su[0] + 2 * hid, L.su[1] = L.sv[0] + 2 * inter, L.sv[1] = L.su[1] + 2 * hid;
  L.su[2] = L.sv[1] + 2 * inter, L.sv[2] = L.su[2] + 2 * inter;
  L.bytes = (L.sv[2] + 2 * hid + 255) / 256 * 256;
  return L;
}
int moe_fused_grid() { return 256; }
MoePlan moe_fused_plan(int, int, int, int, int, bool, int) { return MoePlan(); }  // no fused plan: the staged path
int moe_fused_slots(int, int, int, int) { return 0; }
size_t moe_fused_q8_index(int, int, int) { return 0; }
bool moe_fused_supported(int, int, int, int, int, int, int, bool) { return false; }
bool moe_q8_supported(int hid, int inter) { return hid % 128 == 0 && inter % 128 == 0 && inter <= 1024; }
bool moe_batch_supported(int, int, int, int, int, int) { return false; }
bool moe_batch_few(int, int, int, int, int) { return false; }
int moe_batch_few_chunks(int, int, int, bool) { return 0; }
size_t moe_batch_few_part(int, int, int) { return 0; }
size_t moe_batch_few_epochs(int, int) { return 0; }
int moe_batch_max_chunks(int, int, int, bool) { return 0; }

}  // namespace ijah
