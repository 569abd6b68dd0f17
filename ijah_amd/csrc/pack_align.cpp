// Pack alignment: a copy of a safetensors pack in which every tensor's data starts at a multiple of `align` bytes of
// its shard (reference core/pack_align.h:1-25 `align_pack`, the `align-pack` command of core/main_cli.mm). Shards
// whose tensors are all aligned already, config.json and any other file are symbolic links to the source; a
// misaligned shard is rewritten: its tensors keep their order of appearance, each data offset is rounded up to the
// alignment, and the header is padded with spaces (allowed by the format) so that the data area starts aligned.
// Every rewritten shard goes to "<name>.part" first, is checked byte for byte against the source and renamed into
// place; a rerun keeps a destination shard that already is such a copy.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cstring>

#include "ijah_exl3.h"
#include "json.h"
#include "pack.h"

namespace ijah {
namespace {

std::string quote(const std::string &s) {
  std::string o = "\"";
  for (const unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += (char)c;
    } else if (c < 0x20) {
      o += strfmt("\\u%04x", c);
    } else {
      o += (char)c;
    }
  }
  return o + "\"";
}
std::string dump(const json::Value &v) {
  switch (v.kind) {
    case json::Value::Null: return "null";
    case json::Value::Bool: return v.b ? "true" : "false";
    case json::Value::Num: return v.inum == (int64_t)v.num ? std::to_string(v.inum) : strfmt("%.17g", v.num);
    case json::Value::Str: return quote(v.str);
    case json::Value::Arr: {
      std::string o = "[";
      for (size_t i = 0; i < v.arr.size(); i++) o += (i ? "," : "") + dump(v.arr[i]);
      return o + "]";
    }
    default: {
      std::string o = "{";
      for (size_t i = 0; i < v.obj.size(); i++) o += (i ? "," : "") + quote(v.obj[i].first) + ":" + dump(v.obj[i].second);
      return o + "}";
    }
  }
}

// one shard's entries as its header lists them (absolute data offsets), plus its metadata object
struct Entry {
  std::string name, dtype;
  std::vector<int64_t> shape;
  uint64_t off = 0, nbytes = 0;
};
struct Shard {
  std::vector<Entry> entries;  // in data order
  json::Value meta;
  uint64_t size = 0;
};
Shard read_shard(const std::string &path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  IJ_CHECK(fd >= 0, "align: cannot open %s", path.c_str());
  struct stat st;
  fstat(fd, &st);
  Shard s;
  s.size = (uint64_t)st.st_size;
  uint64_t hlen = 0;
  const bool ok8 = s.size >= 8 && pread(fd, &hlen, 8, 0) == 8;
  std::string h;
  if (ok8 && hlen <= s.size - 8) {
    h.resize(hlen);
    if (pread(fd, &h[0], hlen, 8) != (ssize_t)hlen) h.clear();
  }
  ::close(fd);
  IJ_CHECK(ok8 && h.size() == hlen && hlen > 0, "align: %s: bad header", path.c_str());
  const json::Value v = json::parse(h);
  IJ_CHECK(v.kind == json::Value::Obj, "align: %s: header is not an object", path.c_str());
  for (auto &kv : v.obj) {
    if (kv.first == "__metadata__") {
      s.meta = kv.second;
      continue;
    }
    const json::Value *dt = kv.second.get("dtype"), *sh = kv.second.get("shape"), *of = kv.second.get("data_offsets");
    IJ_CHECK(dt && sh && of && of->arr.size() == 2, "align: %s: bad entry %s", path.c_str(), kv.first.c_str());
    Entry e;
    e.name = kv.first;
    e.dtype = dt->str;
    for (auto &d : sh->arr) e.shape.push_back(d.inum);
    e.off = 8 + hlen + (uint64_t)of->arr[0].inum;
    e.nbytes = (uint64_t)(of->arr[1].inum - of->arr[0].inum);
    IJ_CHECK(e.off + e.nbytes <= s.size, "align: %s: %s beyond the file", path.c_str(), e.name.c_str());
    s.entries.push_back(e);
  }
  std::sort(s.entries.begin(), s.entries.end(), [](const Entry &a, const Entry &b) { return a.off < b.off; });
  return s;
}

// a read-only mapping of a whole file
struct Map {
  const uint8_t *p = nullptr;
  size_t n = 0;
  explicit Map(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    IJ_CHECK(fd >= 0, "align: cannot open %s", path.c_str());
    struct stat st;
    fstat(fd, &st);
    n = (size_t)st.st_size;
    void *m = n ? mmap(nullptr, n, PROT_READ, MAP_SHARED, fd, 0) : nullptr;
    ::close(fd);
    IJ_CHECK(n == 0 || m != MAP_FAILED, "align: mmap %s failed", path.c_str());
    p = (const uint8_t *)m;
  }
  ~Map() {
    if (p) munmap((void *)p, n);
  }
};

// dst holds the same tensors as src (names, dtypes, shapes, bytes), each at an aligned offset
bool is_aligned_copy(const std::string &src, const Shard &s, const std::string &dst, uint64_t align) {
  struct stat st;
  if (lstat(dst.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) return false;
  Shard d;
  try {
    d = read_shard(dst);
  } catch (const Error &) {
    return false;
  }
  if (d.entries.size() != s.entries.size()) return false;
  const Map ms(src), md(dst);
  for (size_t i = 0; i < s.entries.size(); i++) {
    const Entry &a = s.entries[i], &b = d.entries[i];
    if (a.name != b.name || a.dtype != b.dtype || a.shape != b.shape || a.nbytes != b.nbytes || b.off % align)
      return false;
    if (memcmp(ms.p + a.off, md.p + b.off, a.nbytes) != 0) return false;
  }
  return true;
}

void write_full(int fd, const void *p, size_t n, uint64_t off, const std::string &path) {
  const uint8_t *b = (const uint8_t *)p;
  while (n) {
    const ssize_t k = pwrite(fd, b, std::min<size_t>(n, (size_t)1 << 30), (off_t)off);
    IJ_CHECK(k > 0, "align: write %s: %s", path.c_str(), strerror(errno));
    b += k;
    off += (uint64_t)k;
    n -= (size_t)k;
  }
}

// symbolic link dst -> target (an existing link elsewhere is replaced; a regular file is an error)
void link_to(const std::string &target, const std::string &dst) {
  char cur[PATH_MAX];
  const ssize_t k = readlink(dst.c_str(), cur, sizeof cur - 1);
  if (k >= 0) {
    cur[k] = 0;
    if (target == cur) return;
    IJ_CHECK(unlink(dst.c_str()) == 0, "align: cannot replace %s", dst.c_str());
  } else {
    struct stat st;
    IJ_CHECK(lstat(dst.c_str(), &st) != 0, "align: %s exists and is not a link", dst.c_str());
  }
  IJ_CHECK(symlink(target.c_str(), dst.c_str()) == 0, "align: symlink %s: %s", dst.c_str(), strerror(errno));
}

void rewrite(const std::string &src, const Shard &s, const std::string &dst, uint64_t align, ne_pack_align_stats &st) {
  std::vector<uint64_t> rel(s.entries.size());
  uint64_t cur = 0;
  for (size_t i = 0; i < s.entries.size(); i++) {
    cur = (cur + align - 1) / align * align;
    rel[i] = cur;
    cur += s.entries[i].nbytes;
  }
  std::string h = "{";
  if (s.meta.kind == json::Value::Obj) h += "\"__metadata__\":" + dump(s.meta) + ",";
  for (size_t i = 0; i < s.entries.size(); i++) {
    const Entry &e = s.entries[i];
    std::string shp = "[";
    for (size_t d = 0; d < e.shape.size(); d++) shp += (d ? "," : "") + std::to_string(e.shape[d]);
    h += strfmt("%s%s:{\"dtype\":%s,\"shape\":%s],\"data_offsets\":[%llu,%llu]}", i ? "," : "", quote(e.name).c_str(),
                quote(e.dtype).c_str(), shp.c_str(), (unsigned long long)rel[i],
                (unsigned long long)(rel[i] + e.nbytes));
  }
  h += "}";
  const uint64_t data0 = (8 + h.size() + align - 1) / align * align;
  h.append(data0 - 8 - h.size(), ' ');
  const std::string part = dst + ".part";
  const int fd = ::open(part.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
  IJ_CHECK(fd >= 0, "align: create %s: %s", part.c_str(), strerror(errno));
  const uint64_t hlen = h.size();
  {
    const Map ms(src);
    write_full(fd, &hlen, 8, 0, part);
    write_full(fd, h.data(), h.size(), 8, part);
    for (size_t i = 0; i < s.entries.size(); i++)
      write_full(fd, ms.p + s.entries[i].off, s.entries[i].nbytes, data0 + rel[i], part);
    // the last tensor may end short of a page: size the file exactly
    IJ_CHECK(ftruncate(fd, (off_t)(data0 + cur)) == 0, "align: truncate %s", part.c_str());
  }
  IJ_CHECK(fsync(fd) == 0, "align: fsync %s", part.c_str());
  ::close(fd);
  IJ_CHECK(is_aligned_copy(src, s, part, align), "align: %s does not read back as an aligned copy of %s",
           part.c_str(), src.c_str());
  IJ_CHECK(rename(part.c_str(), dst.c_str()) == 0, "align: rename %s: %s", part.c_str(), strerror(errno));
  st.files_rewritten++;
  st.bytes_written += data0 + cur;
}

}  // namespace
}  // namespace ijah

using namespace ijah;

NE_API int ne_pack_align(const char *src_dir, const char *dst_dir, uint64_t align, int dry_run,
                         ne_pack_align_stats *stats) {
  return c_call([&] {
    IJ_CHECK(src_dir && dst_dir, "align: null directory");
    IJ_CHECK(align >= 1 && align <= (1u << 20), "align: alignment %llu out of range", (unsigned long long)align);
    char real[PATH_MAX];
    IJ_CHECK(realpath(src_dir, real), "align: %s: no such directory", src_dir);
    const std::string src = real;
    ne_pack_align_stats st;
    memset(&st, 0, sizeof st);
    if (!dry_run) {
      IJ_CHECK(mkdir(dst_dir, 0755) == 0 || errno == EEXIST, "align: mkdir %s: %s", dst_dir, strerror(errno));
      IJ_CHECK(realpath(dst_dir, real), "align: %s: not a directory", dst_dir);
      IJ_CHECK(src != real, "align: source and destination are the same directory");
    }
    const std::string dst = dry_run ? std::string() : std::string(real);
    std::vector<std::string> files;
    DIR *d = opendir(src.c_str());
    IJ_CHECK(d, "align: cannot list %s", src.c_str());
    while (dirent *e = readdir(d)) {
      const std::string n = e->d_name;
      if (n != "." && n != ".." && (n.size() < 5 || n.compare(n.size() - 5, 5, ".part") != 0)) files.push_back(n);
    }
    closedir(d);
    std::sort(files.begin(), files.end());
    for (const std::string &n : files) {
      std::string path = src + "/" + n;
      if (realpath(path.c_str(), real)) path = real;
      const bool shard = n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0;
      if (!shard) {
        if (!dry_run) link_to(path, dst + "/" + n);
        continue;
      }
      const Shard s = read_shard(path);
      uint64_t mis = 0;
      for (const Entry &e : s.entries) {
        st.tensors++;
        if (e.off % align) {
          mis++;
          st.misaligned_bytes += e.nbytes;
        }
      }
      st.misaligned_tensors += mis;
      if (dry_run) continue;
      const std::string out = dst + "/" + n;
      if (!mis) {
        link_to(path, out);
        st.files_linked++;
      } else if (is_aligned_copy(path, s, out, align)) {
        st.files_kept++;
      } else {
        unlink(out.c_str());  // a stale copy or link from an earlier run
        rewrite(path, s, out, align, st);
      }
    }
    if (stats) *stats = st;
  });
}
