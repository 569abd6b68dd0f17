// The engine.h C API over HIP: errors, dtypes, device query, HBM buffers, safetensors packs, kernels by name.
// Reference: core/capi.mm (the same entry points over Metal).
#include <dirent.h>
#include <fcntl.h>
#include <limits.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>

#include "json.h"
#include "kernels.h"
#include "pack.h"

namespace ijah {

std::string strfmt(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

static thread_local std::string g_last_error;
void set_last_error(const std::string &msg) { g_last_error = msg; }

bool device_available() {
  static int avail = -1;
  if (avail < 0) {
    int n = 0;
    avail = (hipGetDeviceCount(&n) == hipSuccess && n > 0) ? 1 : 0;
  }
  return avail == 1;
}

void ensure_device() {
  static std::once_flag once;
  static std::string err;
  std::call_once(once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
      err = "no HIP device visible";
      return;
    }
    try {  // kernel attributes before any launch (and so before any stream capture)
      init_batch_attrs();
      init_fused_attrs();
      init_lin_attrs();
      noalloc_scratch();  // the allocation-free linear's scratch address on this device
    } catch (const std::exception &e) {
      err = e.what();
    }
  });
  IJ_CHECK(err.empty(), "%s", err.c_str());
}

hipStream_t stream() {
  static hipStream_t s = nullptr;
  static std::once_flag once;
  ensure_device();
  std::call_once(once, [] {
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) s = nullptr;
  });
  IJ_CHECK(s, "hipStreamCreate failed");
  return s;
}

// ---------------------------------------------------------------------------------------------------- dtypes
static const char *kDtypeNames[] = {"F32", "F16", "BF16", "U8", "U16", "U32", "I32",
                                    "I64", "I8",  "I16",  "U64", "F64", "BOOL"};
static const int kDtypeSizes[] = {4, 2, 2, 1, 2, 4, 4, 8, 1, 2, 8, 8, 1};
const char *dtype_name(int dt) { return (dt >= 0 && dt <= 12) ? kDtypeNames[dt] : "?"; }
int dtype_size(int dt) { return (dt >= 0 && dt <= 12) ? kDtypeSizes[dt] : 0; }
int dtype_from_name(const std::string &s) {
  for (int i = 0; i <= 12; i++)
    if (s == kDtypeNames[i]) return i;
  return -1;
}

// ---------------------------------------------------------------------------------------------------- packs
static std::string read_file(const std::string &path, bool *ok) {
  std::ifstream f(path, std::ios::binary);
  *ok = (bool)f;
  if (!f) return "";
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

std::unique_ptr<Pack> Pack::open(const std::string &dir_in) {
  char real[PATH_MAX];
  IJ_CHECK(realpath(dir_in.c_str(), real), "pack: %s: no such directory", dir_in.c_str());
  auto p = std::unique_ptr<Pack>(new Pack());
  p->dir_ = real;
  bool ok = false;
  p->config_ = read_file(p->dir_ + "/config.json", &ok);
  if (!ok) p->config_ = "{}";
  std::vector<std::string> shards;
  DIR *d = opendir(real);
  IJ_CHECK(d, "pack: cannot list %s", real);
  while (dirent *e = readdir(d)) {
    const std::string n = e->d_name;
    if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) shards.push_back(n);
  }
  closedir(d);
  std::sort(shards.begin(), shards.end());
  IJ_CHECK(!shards.empty(), "pack: no .safetensors files in %s", real);
  for (const std::string &sh : shards) {
    std::string path = p->dir_ + "/" + sh;
    char rp[PATH_MAX];
    if (realpath(path.c_str(), rp)) path = rp;
    const int fd = ::open(path.c_str(), O_RDONLY);
    IJ_CHECK(fd >= 0, "pack: cannot open %s", path.c_str());
    struct stat st;
    fstat(fd, &st);
    const size_t len = (size_t)st.st_size;
    void *m = len ? mmap(nullptr, len, PROT_READ, MAP_SHARED, fd, 0) : nullptr;
    ::close(fd);
    IJ_CHECK(len == 0 || m != MAP_FAILED, "pack: mmap %s failed", path.c_str());
    const int fi = (int)p->files_.size();
    p->files_.push_back(path);
    p->maps_.emplace_back(m, len);
    IJ_CHECK(len >= 8, "pack: %s: too short", path.c_str());
    uint64_t hlen = 0;
    memcpy(&hlen, m, 8);
    IJ_CHECK(hlen <= len - 8, "pack: %s: header length %llu beyond file", path.c_str(), (unsigned long long)hlen);
    const json::Value h = json::parse(std::string((const char *)m + 8, hlen));
    IJ_CHECK(h.kind == json::Value::Obj, "pack: %s: header is not an object", path.c_str());
    const uint64_t data0 = 8 + hlen;
    for (auto &kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      const json::Value &t = kv.second;
      const json::Value *dt = t.get("dtype"), *sh = t.get("shape"), *of = t.get("data_offsets");
      IJ_CHECK(dt && sh && of && of->arr.size() == 2, "pack: %s: bad entry %s", path.c_str(), kv.first.c_str());
      TensorInfo ti;
      ti.dtype = dtype_from_name(dt->str);
      IJ_CHECK(ti.dtype >= 0, "pack: %s: dtype %s", kv.first.c_str(), dt->str.c_str());
      IJ_CHECK((int)sh->arr.size() <= NE_MAX_DIMS, "pack: %s: too many dims", kv.first.c_str());
      ti.ndim = (int)sh->arr.size();
      for (int i = 0; i < ti.ndim; i++) ti.shape[i] = sh->arr[i].inum;
      const uint64_t a = (uint64_t)of->arr[0].inum, b = (uint64_t)of->arr[1].inum;
      IJ_CHECK(b >= a && data0 + b <= len, "pack: %s: data beyond file", kv.first.c_str());
      ti.nbytes = b - a;
      IJ_CHECK(ti.nbytes == (uint64_t)ti.numel() * dtype_size(ti.dtype), "pack: %s: size mismatch",
               kv.first.c_str());
      ti.file = fi;
      ti.file_offset = data0 + a;
      ti.host = (const char *)m + data0 + a;
      IJ_CHECK(!p->tensors_.count(kv.first), "pack: tensor %s in two shards", kv.first.c_str());
      p->tensors_[kv.first] = ti;
    }
  }
  for (auto &kv : p->tensors_) p->names_.push_back(kv.first);  // std::map: sorted by name
  return p;
}

Pack::~Pack() {
  for (auto &m : maps_)
    if (m.first) munmap(m.first, m.second);
}

const TensorInfo *Pack::info(const std::string &name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorInfo &Pack::need(const std::string &name, int dtype, std::initializer_list<int64_t> shape) const {
  const TensorInfo *t = info(name);
  IJ_CHECK(t, "pack: no tensor %s", name.c_str());
  IJ_CHECK(dtype < 0 || t->dtype == dtype, "pack: %s is %s, expected %s", name.c_str(), dtype_name(t->dtype),
           dtype_name(dtype));
  if (shape.size()) {
    bool ok = (int)shape.size() == t->ndim;
    int i = 0;
    for (int64_t s : shape) {
      if (ok && s >= 0 && t->shape[i] != s) ok = false;
      i++;
    }
    std::string got;
    for (int k = 0; k < t->ndim; k++) got += (k ? "," : "") + std::to_string(t->shape[k]);
    IJ_CHECK(ok, "pack: %s has shape [%s]", name.c_str(), got.c_str());
  }
  return *t;
}

}  // namespace ijah

using namespace ijah;

ne_buf::~ne_buf() {
  if (dev && !external) (void)hipFree(dev);
  free(host);
  free(snap);
}

namespace ijah {
void mirror_push(const ne_buf *cb) {
  ne_buf *b = const_cast<ne_buf *>(cb);
  if (!b || !b->host || !b->snap || b->readonly || !b->size) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream(), &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
  const uint8_t *h = (const uint8_t *)b->host;
  uint8_t *sn = (uint8_t *)b->snap;
  const uint64_t n = b->size;
  bool synced = false;
  uint64_t i = 0;
  while (i < n) {
    // next changed byte (8 bytes at a time), then the end of the run of changed 8-byte words
    while (i + 8 <= n && memcmp(h + i, sn + i, 8) == 0) i += 8;
    while (i < n && h[i] == sn[i]) i++;
    if (i >= n) break;
    uint64_t e = i + 1;
    while (e < n) {
      const uint64_t w = std::min<uint64_t>(8, n - e);
      if (memcmp(h + e, sn + e, w) == 0) break;
      e += w;
    }
    while (e > i + 1 && h[e - 1] == sn[e - 1]) e--;  // trim unchanged bytes at the end of the run
    if (!synced) {
      IJ_HIP(hipStreamSynchronize(stream()));
      synced = true;
    }
    IJ_HIP(hipMemcpy((uint8_t *)b->dev + i, h + i, e - i, hipMemcpyHostToDevice));
    memcpy(sn + i, h + i, e - i);
    i = e;
  }
}
void *ne_dev(const ne_buf *b) {
  mirror_push(b);
  return b ? b->dev : nullptr;
}
}  // namespace ijah

static ne_buf *new_device_buf(uint64_t n) {
  ensure_device();
  auto b = std::make_unique<ne_buf>();
  b->size = n;
  if (n) {
    IJ_HIP(hipMalloc(&b->dev, n));
    IJ_HIP(hipMemsetAsync(b->dev, 0, n, stream()));
    IJ_HIP(hipStreamSynchronize(stream()));
  }
  return b.release();
}

extern "C" {

NE_API int ne_abi_version(void) { return NE_ABI_VERSION; }
NE_API const char *ne_last_error(void) { return g_last_error.c_str(); }
NE_API const char *ne_dtype_name(int t) { return dtype_name(t); }
NE_API int ne_dtype_size(int t) { return dtype_size(t); }

NE_API int ne_device_query(ne_device_info *out) {
  return c_call([&] {
    IJ_CHECK(out, "null out");
    ensure_device();
    int dev = 0;
    IJ_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    IJ_HIP(hipGetDeviceProperties(&p, dev));
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s (%s)", p.name, p.gcnArchName);
    out->has_nax = 1;
    out->has_metal4 = 0;
    out->max_buffer_length = p.totalGlobalMem;
    out->recommended_working_set = p.totalGlobalMem;
    out->max_threadgroup_memory = p.maxSharedMemoryPerMultiProcessor;
    snprintf(out->backend, sizeof out->backend, "hip");
  });
}

NE_API ne_buf *ne_alloc(uint64_t nbytes) {
  ne_buf *h = nullptr;
  c_call([&] { h = new_device_buf(nbytes); });
  return h;
}
NE_API void ne_free(ne_buf *b) {
  if (b && b->owned) delete b;
}
NE_API uint64_t ne_buf_size(const ne_buf *b) { return b ? b->size : 0; }
NE_API void *ne_buf_contents(const ne_buf *b) {
  void *r = nullptr;
  c_call([&] {
    IJ_CHECK(b, "null buffer");
    ne_buf *m = const_cast<ne_buf *>(b);
    mirror_push(m);  // writes made through an earlier pointer reach the device first
    if (!m->host) m->host = calloc(1, m->size ? m->size : 1);
    if (!m->snap) m->snap = calloc(1, m->size ? m->size : 1);
    IJ_CHECK(m->host && m->snap, "host mirror allocation failed");
    if (m->size) {
      IJ_HIP(hipStreamSynchronize(stream()));
      IJ_HIP(hipMemcpy(m->host, m->dev, m->size, hipMemcpyDeviceToHost));
      memcpy(m->snap, m->host, m->size);
    }
    r = m->host;
  });
  return r;
}
NE_API uint64_t ne_buf_gpu_address(const ne_buf *b) { return b ? (uint64_t)(uintptr_t)b->dev : 0; }
NE_API int ne_upload(ne_buf *b, uint64_t offset, const void *src, uint64_t n) {
  return c_call([&] {
    IJ_CHECK(b && offset <= b->size && n <= b->size - offset, "upload out of range");
    IJ_CHECK(!b->readonly, "upload into a pack tensor (read-only)");
    IJ_CHECK(src || n == 0, "null source");
    if (!n) return;
    mirror_push(b);
    IJ_HIP(hipStreamSynchronize(stream()));
    IJ_HIP(hipMemcpy((char *)b->dev + offset, src, n, hipMemcpyHostToDevice));
  });
}
NE_API int ne_download(const ne_buf *b, uint64_t offset, void *dst, uint64_t n) {
  return c_call([&] {
    IJ_CHECK(b && offset <= b->size && n <= b->size - offset, "download out of range");
    IJ_CHECK(dst || n == 0, "null destination");
    if (!n) return;
    mirror_push(b);
    IJ_HIP(hipStreamSynchronize(stream()));
    IJ_HIP(hipMemcpy(dst, (const char *)b->dev + offset, n, hipMemcpyDeviceToHost));
  });
}
NE_API int ne_buf_flush(ne_buf *b) {
  return c_call([&] {
    IJ_CHECK(b, "null buffer");
    IJ_CHECK(!b->readonly, "flush into a pack tensor (read-only)");
    if (!b->host || !b->size) return;
    IJ_HIP(hipStreamSynchronize(stream()));
    IJ_HIP(hipMemcpy(b->dev, b->host, b->size, hipMemcpyHostToDevice));
    if (b->snap) memcpy(b->snap, b->host, b->size);
  });
}
NE_API int ne_sync(void) {
  return c_call([&] { IJ_HIP(hipStreamSynchronize(stream())); });
}
NE_API void *ne_stream(void) {
  void *s = nullptr;
  c_call([&] { s = (void *)stream(); });
  return s;
}

NE_API ne_pack *ne_pack_open(const char *dir) {
  ne_pack *p = nullptr;
  c_call([&] {
    IJ_CHECK(dir, "null dir");
    auto u = std::make_unique<ne_pack>();
    u->pack = Pack::open(dir);
    p = u.release();
  });
  return p;
}
NE_API void ne_pack_close(ne_pack *p) {
  if (!p) return;
  for (auto &kv : p->bufs) delete kv.second;
  delete p;
}
NE_API const char *ne_pack_config_json(const ne_pack *p) { return p ? p->pack->config().c_str() : nullptr; }
NE_API int64_t ne_pack_num_tensors(const ne_pack *p) { return p ? (int64_t)p->pack->names().size() : -1; }
NE_API const char *ne_pack_tensor_name(const ne_pack *p, int64_t i) {
  if (!p || i < 0 || i >= (int64_t)p->pack->names().size()) {
    set_last_error("tensor index out of range");
    return nullptr;
  }
  return p->pack->names()[(size_t)i].c_str();
}

// Device copies of pack tensors are made on the first ne_tensor_info (tensors up to 1 GiB; larger ones report
// buf = NULL, like the reference's tensors beyond max_buffer_length, and are reached with ne_pack_view_rows).
static const uint64_t kMaxTensorCopy = 1ull << 30;

NE_API int ne_tensor_info(const ne_pack *p, const char *name, ne_tensor_desc *out) {
  return c_call([&] {
    IJ_CHECK(p && name && out, "null argument");
    const TensorInfo *ti = p->pack->info(name);
    IJ_CHECK(ti, "no tensor %s", name);
    memset(out, 0, sizeof *out);
    out->dtype = ti->dtype;
    out->ndim = ti->ndim;
    for (int i = 0; i < ti->ndim; i++) out->shape[i] = ti->shape[i];
    out->nbytes = ti->nbytes;
    out->file = p->pack->file(ti->file).c_str();
    out->file_offset = ti->file_offset;
    out->host = ti->host;
    if (ti->nbytes == 0 || ti->nbytes > kMaxTensorCopy || !device_available()) return;
    ne_pack *mp = const_cast<ne_pack *>(p);
    auto it = mp->bufs.find(name);
    if (it == mp->bufs.end()) {
      std::unique_ptr<ne_buf> b(new_device_buf(ti->nbytes));
      IJ_HIP(hipMemcpy(b->dev, ti->host, ti->nbytes, hipMemcpyHostToDevice));
      b->owned = false;
      b->readonly = true;
      it = mp->bufs.emplace(name, b.release()).first;
    }
    out->buf = it->second;
    out->buf_offset = 0;
  });
}

NE_API ne_buf *ne_pack_view_rows(const ne_pack *p, const char *name, int64_t row0, int64_t nrows, uint64_t *offset) {
  ne_buf *h = nullptr;
  c_call([&] {
    IJ_CHECK(p && name, "null argument");
    const TensorInfo *ti = p->pack->info(name);
    IJ_CHECK(ti, "no tensor %s", name);
    IJ_CHECK(ti->ndim >= 1 && row0 >= 0 && nrows >= 0 && row0 + nrows <= ti->shape[0], "rows out of range");
    const uint64_t row_bytes = ti->shape[0] ? ti->nbytes / (uint64_t)ti->shape[0] : 0;
    std::unique_ptr<ne_buf> b(new_device_buf(row_bytes * (uint64_t)nrows));
    if (nrows)
      IJ_HIP(hipMemcpy(b->dev, (const char *)ti->host + row_bytes * (uint64_t)row0, row_bytes * (uint64_t)nrows,
                       hipMemcpyHostToDevice));
    b->readonly = true;
    if (offset) *offset = 0;
    h = b.release();
  });
  return h;
}

NE_API int ne_kernel_exists(const char *fn) {
  int r = -1;
  c_call([&] { r = find_kernel(fn ? fn : "", nullptr, 0) ? 1 : 0; });
  return r;
}

NE_API int ne_run_kernel(const char *fn, const ne_fconst *fc, int nfc, const ne_arg *args, int nargs,
                         const uint32_t grid[3], const uint32_t tg[3], uint32_t tg_mem, int reps, const char *backend,
                         double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(fn && grid && tg && (nargs == 0 || args) && (nfc == 0 || fc), "null argument");
    IJ_CHECK(!backend || !*backend || !strcmp(backend, "hip"), "backend %s: only \"hip\" exists here", backend);
    const KernelEntry *k = find_kernel(fn, fc, nfc);
    IJ_CHECK(k, "no kernel %s with these function constants", fn);
    IJ_CHECK((int)k->arg_sizes.size() == nargs, "%s takes %zu arguments, got %d", fn, k->arg_sizes.size(), nargs);
    IJ_CHECK(tg[0] * tg[1] * tg[2] > 0 && tg[0] * tg[1] * tg[2] <= 1024, "%s: workgroup size out of range", fn);
    std::vector<void *> ptrs(nargs);
    std::vector<void *> addr(nargs);
    for (int i = 0; i < nargs; i++) {
      if (args[i].bytes) {
        IJ_CHECK(args[i].nbytes == k->arg_sizes[i], "%s: argument %d is %u bytes, kernel expects %u", fn, i,
                 args[i].nbytes, k->arg_sizes[i]);
        addr[i] = const_cast<void *>(args[i].bytes);
      } else {
        IJ_CHECK(args[i].buf && args[i].buf->dev, "argument %d: null buffer", i);
        mirror_push(args[i].buf);
        IJ_CHECK(k->arg_sizes[i] == sizeof(void *), "%s: argument %d must be inline bytes", fn, i);
        IJ_CHECK(args[i].offset <= args[i].buf->size, "argument %d: offset beyond buffer", i);
        ptrs[i] = (char *)args[i].buf->dev + args[i].offset;
        addr[i] = &ptrs[i];
      }
    }
    hipStream_t s = stream();
    hipEvent_t e0, e1;
    IJ_HIP(hipEventCreate(&e0));
    IJ_HIP(hipEventCreate(&e1));
    IJ_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < std::max(reps, 1); r++)
      IJ_HIP(hipLaunchKernel(k->fn, dim3(grid[0], grid[1], grid[2]), dim3(tg[0], tg[1], tg[2]), addr.data(), tg_mem,
                             s));
    IJ_HIP(hipEventRecord(e1, s));
    IJ_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    IJ_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (gpu_ms) *gpu_ms = ms;
  });
}

}  // extern "C"
