// Safetensors shard reader for the expert store's misses.  A shard's header
// is parsed once at open; an expert's slice of a [E, ...] tensor is a
// contiguous byte range along dimension 0.  Reads use pread from a small
// pool of spinning threads (the page cache is copied by the kernel: no page
// faults on a user mapping, several threads share the copy).
//
// klc_st_load_mxfp4_packed goes from the file to the packed row-tile layout
// in HBM in one pass: chunks of 64-row tiles are read into the slots of a
// ring in pinned host memory, and a pack kernel reads each slot over PCIe
// and writes its tiles.  There is no SDMA copy: on MI355X an H2D copy
// followed by a kernel on the same stream ran at 10 GB/s (the engine
// hand-off), a kernel reading pinned memory at 52 GB/s.  The ring outlives
// the call, so a load returns once its packs are enqueued and the next
// load's reads overlap them.  klc_st_copy_rows_* stage plain byte ranges
// through the same kind of ring with hipMemcpyAsync.
//
// Replaces the per-miss safe_open(...).get_slice(name)[expert] ->
// .contiguous().pin_memory() -> .to(device) chain of mxfp4_expert.py:478-525
// (and streamed_loader.py:43-82's index use).  File format: 8-byte
// little-endian header length N, N bytes of JSON mapping each tensor name to
// {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the
// byte after the header), an optional "__metadata__" object, then the data.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "klc_common.h"

namespace klc {
namespace {

struct StTensor {
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;  // byte range relative to the data section
};

struct StFile {
  int fd = -1;
  int64_t size = 0;
  int64_t data_start = 0;
  std::map<std::string, StTensor> tensors;
};

// The safetensors format caps the header at 100 MB.
constexpr int64_t kMaxHeaderBytes = 100000000;
// Each reader thread takes at least this much of a range.
constexpr int64_t kMinSliceBytes = 128 << 10;

// Reads [off, off + n) of fd into dst; false (errno set) on an error or EOF.
bool pread_all(int fd, void* dst, int64_t n, int64_t off) {
  uint8_t* d = static_cast<uint8_t*>(dst);
  while (n > 0) {
    const ssize_t r = pread(fd, d, (size_t)std::min<int64_t>(n, 1 << 30), (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) {
      if (r == 0) errno = EIO;
      return false;
    }
    d += r;
    off += r;
    n -= r;
  }
  return true;
}

// A fixed pool of reader threads (created on first use, kept for the life of
// the process).  run(n, fn) calls fn(0..n-1) on the workers and the caller
// and returns when all have finished; concurrent callers take turns.  A job
// is published through one 64-bit ticket, (generation << 32) | next slice:
// a slice is claimed by a compare-exchange that also checks the generation.
// Before the next job is written the finished one's ticket is retired (slice
// index past any count), so a worker holding a finished job's generation
// claims nothing.  Between
// jobs a worker spins for kSpinNs before it sleeps, so the chunks of one
// load, tens of microseconds apart, find it awake.  In a forked child the
// workers do not exist, so the caller runs every slice.
class ReadPool {
 public:
  static ReadPool& get() {
    static ReadPool* pool = new ReadPool((int)std::min<unsigned>(kMaxReaders, std::max(1u, std::thread::hardware_concurrency())));
    return *pool;
  }
  int threads() const { return getpid() == pid_ ? (int)workers_ + 1 : 1; }

  void run(int n, const std::function<void(int)>& fn) {
    if (n <= 1 || getpid() != pid_) {
      for (int i = 0; i < n; ++i) fn(i);
      return;
    }
    std::lock_guard<std::mutex> turn(run_m_);
    // Retire the finished job first: its ticket's slice index becomes
    // kRetired, above any slice count, so a worker still holding that
    // generation claims nothing, whatever n_ it reads while the new job is
    // written (a stale compare-exchange fails on the changed ticket).
    const uint64_t old_gen = ticket_.load(std::memory_order_relaxed) >> 32;
    ticket_.store((old_gen << 32) | kRetired, std::memory_order_seq_cst);
    job_ = &fn;
    n_.store(n, std::memory_order_relaxed);
    unfinished_.store(n, std::memory_order_relaxed);
    const uint64_t gen = old_gen + 1;
    ticket_.store(gen << 32, std::memory_order_seq_cst);
    if (sleepers_.load(std::memory_order_seq_cst) > 0) {
      std::lock_guard<std::mutex> g(m_);
      cv_work_.notify_all();
    }
    work(gen);
    while (unfinished_.load(std::memory_order_acquire) != 0) {
    }
  }

 private:
  static constexpr unsigned kMaxReaders = 16;
  static constexpr int64_t kSpinNs = 200000;
  static constexpr uint64_t kRetired = 0xffffffffu;

  explicit ReadPool(int threads) : pid_(getpid()), workers_(threads - 1) {
    for (unsigned i = 0; i < workers_; ++i) std::thread([this] { loop(); }).detach();
  }
  // claims and runs slices of generation gen until none is left
  void work(uint64_t gen) {
    uint64_t t = ticket_.load(std::memory_order_acquire);
    for (;;) {
      if ((t >> 32) != gen || (int64_t)(t & 0xffffffffu) >= n_.load(std::memory_order_relaxed)) return;
      if (!ticket_.compare_exchange_weak(t, t + 1, std::memory_order_acq_rel, std::memory_order_acquire)) continue;
      (*job_)((int)(t & 0xffffffffu));
      unfinished_.fetch_sub(1, std::memory_order_acq_rel);
      t = ticket_.load(std::memory_order_acquire);
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      uint64_t gen = ticket_.load(std::memory_order_acquire) >> 32;
      if (gen == seen) {
        const auto until = std::chrono::steady_clock::now() + std::chrono::nanoseconds(kSpinNs);
        for (int spin = 0; gen == seen; ++spin) {
          if ((spin & 255) == 255 && std::chrono::steady_clock::now() > until) break;
          gen = ticket_.load(std::memory_order_acquire) >> 32;
        }
      }
      if (gen == seen) {
        std::unique_lock<std::mutex> g(m_);
        sleepers_.fetch_add(1, std::memory_order_seq_cst);
        cv_work_.wait(g, [&] { return (ticket_.load(std::memory_order_seq_cst) >> 32) != seen; });
        sleepers_.fetch_sub(1, std::memory_order_relaxed);
        gen = ticket_.load(std::memory_order_acquire) >> 32;
      }
      seen = gen;
      work(gen);
    }
  }

  const pid_t pid_;
  const unsigned workers_;
  std::mutex run_m_, m_;
  std::condition_variable cv_work_;
  const std::function<void(int)>* job_ = nullptr;
  std::atomic<uint64_t> ticket_{0};
  std::atomic<int> n_{0}, unfinished_{0}, sleepers_{0};
};

// Reads [off, off + n) of the file into dst with the pool; 0 or the errno
// of the first failed slice.
int parallel_read(const StFile* f, void* dst, int64_t n, int64_t off) {
  if (n <= 0) return 0;
  ReadPool& pool = ReadPool::get();
  const int64_t max_slices = std::max<int64_t>(1, n / kMinSliceBytes);
  const int slices = (int)std::min<int64_t>(pool.threads(), max_slices);
  const int64_t per = (n + slices - 1) / slices;
  std::mutex em;
  int err = 0;
  pool.run(slices, [&](int i) {
    const int64_t b = i * per, e = std::min<int64_t>(n, b + per);
    if (b < e && !pread_all(f->fd, static_cast<uint8_t*>(dst) + b, e - b, off + b)) {
      const int code = errno;
      std::lock_guard<std::mutex> g(em);
      if (err == 0) err = code;
    }
  });
  return err;
}

// A JSON reader for the header: objects, arrays, strings (all escapes,
// \u as UTF-8), integers, and skipping of any other value.
class Json {
 public:
  Json(const char* p, const char* end) : p_(p), end_(end) {}

  bool parse_header(std::map<std::string, StTensor>& out) {
    ws();
    if (!eat('{')) return false;
    ws();
    if (eat('}')) return true;
    for (;;) {
      std::string key;
      ws();
      if (!string(key)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (key == "__metadata__") {
        if (!skip()) return false;
      } else {
        StTensor t;
        if (!tensor(t)) return false;
        out[key] = t;
      }
      ws();
      if (eat(',')) continue;
      return eat('}');
    }
  }

 private:
  const char* p_;
  const char* end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool eat(char c) {
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  static void utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xc0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      s += (char)(0xe0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    } else {
      s += (char)(0xf0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3f));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    }
  }
  bool hex4(uint32_t& v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& s) {
    if (!eat('"')) return false;
    while (p_ < end_) {
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return false;
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xd800 && cp < 0xdc00) {  // surrogate pair
            uint32_t lo;
            if (!eat('\\') || !eat('u') || !hex4(lo) || lo < 0xdc00 || lo >= 0xe000) return false;
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          utf8(s, cp);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool integer(int64_t& v) {
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
    v = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      if (v > (INT64_MAX - 9) / 10) return false;
      v = v * 10 + (*p_++ - '0');
    }
    return true;
  }
  bool int_array(std::vector<int64_t>& a) {
    if (!eat('[')) return false;
    ws();
    if (eat(']')) return true;
    for (;;) {
      int64_t v;
      ws();
      if (!integer(v)) return false;
      a.push_back(v);
      ws();
      if (eat(',')) continue;
      return eat(']');
    }
  }
  bool tensor(StTensor& t) {
    if (!eat('{')) return false;
    bool have_dtype = false, have_shape = false, have_off = false;
    ws();
    if (!eat('}')) {
      for (;;) {
        std::string key;
        ws();
        if (!string(key)) return false;
        ws();
        if (!eat(':')) return false;
        ws();
        if (key == "dtype") {
          if (!string(t.dtype)) return false;
          have_dtype = true;
        } else if (key == "shape") {
          if (!int_array(t.shape)) return false;
          have_shape = true;
        } else if (key == "data_offsets") {
          std::vector<int64_t> o;
          if (!int_array(o) || o.size() != 2 || o[1] < o[0]) return false;
          t.begin = o[0];
          t.end = o[1];
          have_off = true;
        } else if (!skip()) {
          return false;
        }
        ws();
        if (eat(',')) continue;
        if (!eat('}')) return false;
        break;
      }
    }
    return have_dtype && have_shape && have_off;
  }
  bool skip(int depth = 0) {  // any JSON value, nested at most 64 deep
    ws();
    if (p_ >= end_ || depth > 64) return false;
    if (*p_ == '"') {
      std::string s;
      return string(s);
    }
    if (*p_ == '{' || *p_ == '[') {
      const char close = *p_ == '{' ? '}' : ']';
      const bool obj = *p_ == '{';
      ++p_;
      ws();
      if (eat(close)) return true;
      for (;;) {
        ws();
        if (obj) {
          std::string k;
          if (!string(k)) return false;
          ws();
          if (!eat(':')) return false;
        }
        if (!skip(depth + 1)) return false;
        ws();
        if (eat(',')) continue;
        return eat(close);
      }
    }
    // number, true, false, null
    const char* s = p_;
    while (p_ < end_ && *p_ != ',' && *p_ != '}' && *p_ != ']' && *p_ != ' ' && *p_ != '\n' && *p_ != '\r' &&
           *p_ != '\t')
      ++p_;
    return p_ > s;
  }
};

int64_t dtype_bytes(const std::string& d) {
  if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  return 0;
}

// A tensor and the file range of rows [first, first + count) along dim 0.
int row_range(StFile* f, const char* name, int64_t first, int64_t count, int64_t* offset, int64_t* bytes) {
  KLC_REQUIRE(f && name, KLC_ERR_ARGUMENT, "safetensors: null handle or name");
  const auto it = f->tensors.find(name);
  KLC_REQUIRE(it != f->tensors.end(), KLC_ERR_ARGUMENT, "safetensors: no tensor named '%s'", name);
  const StTensor& t = it->second;
  KLC_REQUIRE(!t.shape.empty(), KLC_ERR_SHAPE, "safetensors: '%s' is a scalar", name);
  KLC_REQUIRE(dtype_bytes(t.dtype) > 0, KLC_ERR_UNSUPPORTED, "safetensors: '%s' has dtype %s, whose rows are not sliced",
              name, t.dtype.c_str());
  const int64_t rows = t.shape[0];
  KLC_REQUIRE(first >= 0 && count >= 0 && first + count <= rows, KLC_ERR_SHAPE,
              "safetensors: rows [%lld, %lld) outside the %lld rows of '%s'", (long long)first,
              (long long)(first + count), (long long)rows, name);
  const int64_t row_bytes = rows > 0 ? (t.end - t.begin) / rows : 0;
  *offset = f->data_start + t.begin + first * row_bytes;
  *bytes = count * row_bytes;
  return KLC_OK;
}

}  // namespace
}  // namespace klc

using namespace klc;

extern "C" int klc_st_open(const char* path, void** handle) {
  KLC_REQUIRE(path && handle, KLC_ERR_ARGUMENT, "klc_st_open: null argument");
  *handle = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  KLC_REQUIRE(fd >= 0, KLC_ERR_ARGUMENT, "klc_st_open: cannot open %s: %s", path, strerror(errno));
  StFile* f = new StFile;
  f->fd = fd;
  struct stat st;
  uint8_t len[8];
  int rc = KLC_OK;
  if (fstat(fd, &st) != 0 || st.st_size < 8 || !pread_all(fd, len, 8, 0)) {
    rc = set_error(KLC_ERR_SHAPE, "klc_st_open: %s is not a safetensors file (too short)", path);
  } else {
    f->size = (int64_t)st.st_size;
    uint64_t n = 0;
    for (int i = 0; i < 8; ++i) n |= (uint64_t)len[i] << (8 * i);
    if (n > (uint64_t)(f->size - 8) || n > (uint64_t)kMaxHeaderBytes) {
      rc = set_error(KLC_ERR_SHAPE, "klc_st_open: %s: header of %llu bytes exceeds the file or 100 MB", path,
                     (unsigned long long)n);
    } else {
      f->data_start = 8 + (int64_t)n;
      std::vector<char> h((size_t)n);
      if (!pread_all(fd, h.data(), (int64_t)n, 8)) {
        rc = set_error(KLC_ERR_ARGUMENT, "klc_st_open: cannot read %s: %s", path, strerror(errno));
      } else if (!Json(h.data(), h.data() + n).parse_header(f->tensors)) {
        rc = set_error(KLC_ERR_SHAPE, "klc_st_open: %s: malformed header", path);
      } else {
        const int64_t data = f->size - f->data_start;
        for (const auto& kv : f->tensors) {
          const StTensor& t = kv.second;
          int64_t elems = 1;
          for (int64_t d : t.shape) elems = d >= 0 && (d == 0 || elems <= INT64_MAX / d) ? elems * d : -1;
          const int64_t eb = dtype_bytes(t.dtype);
          if (t.end > data || elems < 0 || elems > (INT64_MAX >> 3) || (eb > 0 && elems * eb != t.end - t.begin)) {
            rc = set_error(KLC_ERR_SHAPE, "klc_st_open: %s: tensor '%s' has inconsistent offsets", path,
                           kv.first.c_str());
            break;
          }
        }
      }
    }
  }
  if (rc != KLC_OK) {
    close(fd);
    delete f;
    return rc;
  }
  *handle = f;
  return KLC_OK;
}

extern "C" int klc_st_close(void* handle) {
  StFile* f = static_cast<StFile*>(handle);
  if (f == nullptr) return KLC_OK;
  close(f->fd);
  delete f;
  return KLC_OK;
}

extern "C" int klc_st_tensor_info(void* handle, const char* name, char* dtype, int64_t* shape, int* ndim,
                                  int64_t* data_offset, int64_t* nbytes) {
  StFile* f = static_cast<StFile*>(handle);
  KLC_REQUIRE(f && name && dtype && shape && ndim && data_offset && nbytes, KLC_ERR_ARGUMENT,
              "klc_st_tensor_info: null argument");
  const auto it = f->tensors.find(name);
  KLC_REQUIRE(it != f->tensors.end(), KLC_ERR_ARGUMENT, "safetensors: no tensor named '%s'", name);
  const StTensor& t = it->second;
  KLC_REQUIRE(t.shape.size() <= 8, KLC_ERR_UNSUPPORTED, "safetensors: '%s' has more than 8 dimensions", name);
  snprintf(dtype, 16, "%s", t.dtype.c_str());
  *ndim = (int)t.shape.size();
  for (size_t i = 0; i < t.shape.size(); ++i) shape[i] = t.shape[i];
  *data_offset = f->data_start + t.begin;
  *nbytes = t.end - t.begin;
  return KLC_OK;
}

extern "C" int klc_st_read_rows(void* handle, const char* name, int64_t first, int64_t count, void* dst) {
  StFile* f = static_cast<StFile*>(handle);
  int64_t off, bytes;
  const int rc = row_range(f, name, first, count, &off, &bytes);
  if (rc) return rc;
  KLC_REQUIRE(dst || bytes == 0, KLC_ERR_ARGUMENT, "klc_st_read_rows: null destination");
  const int err = parallel_read(f, dst, bytes, off);
  KLC_REQUIRE(err == 0, KLC_ERR_ARGUMENT, "klc_st_read_rows: read of '%s' failed: %s", name, strerror(err));
  return KLC_OK;
}

namespace klc {
namespace {

// Staging slots of the packing loads: small enough that the first slot's
// read is short and the pack kernels over PCIe, not the reads, set the pace.
constexpr int64_t kSlotBytes = 2 << 20;
// Staging slots of the plain row copies.  A host-to-device copy moves
// 45 GB/s in 2 MiB pieces against 53 GB/s in 8 MiB pieces (57 GB/s for one
// 64 MiB copy) on MI355X over PCIe 5; the first chunk of a load is a quarter
// slot, so its read stays short.
constexpr int64_t kCopySlotBytes = 8 << 20;
constexpr int kMaxSlots = 64;

// Completion events of the staging slots, per calling thread and device:
// created on first use and kept, so a call creates none.
hipError_t slot_events(int n, hipEvent_t** out) {
  struct PerDevice {
    int device;
    std::vector<hipEvent_t> ev;
  };
  static thread_local std::vector<PerDevice> cache;
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  PerDevice* pd = nullptr;
  for (auto& c : cache)
    if (c.device == device) pd = &c;
  if (pd == nullptr) {
    cache.push_back(PerDevice{device, {}});
    pd = &cache.back();
  }
  while ((int)pd->ev.size() < n) {
    hipEvent_t e;
    err = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (err != hipSuccess) return err;
    pd->ev.push_back(e);
  }
  *out = pd->ev.data();
  return hipSuccess;
}

// The slot ring of one pinned staging buffer on one device, kept across
// calls of klc_st_load_mxfp4_packed: which slots still have a pack in flight
// (used + ev) and where the next chunk goes.  A call with another slot
// layout first waits for every slot.  The registry is global, so any thread
// may wait for or release a buffer's ring; one buffer is filled by one
// thread at a time.
struct Ring {
  int slots = 0;
  int64_t slot_bytes = 0;
  int next = 0;
  bool used[kMaxSlots] = {};
  hipEvent_t ev[kMaxSlots] = {};
};
std::mutex g_rings_m;
std::map<std::pair<const void*, int>, Ring*> g_rings;

Ring* ring_of(const void* staging, int device) {
  std::lock_guard<std::mutex> g(g_rings_m);
  Ring*& r = g_rings[{staging, device}];
  if (r == nullptr) r = new Ring;
  return r;
}

hipError_t ring_drain(Ring* r) {
  hipError_t first = hipSuccess;
  for (int b = 0; b < kMaxSlots; ++b) {
    if (!r->used[b]) continue;
    const hipError_t e = hipEventSynchronize(r->ev[b]);
    if (e != hipSuccess && first == hipSuccess) first = e;
    r->used[b] = false;
  }
  return first;
}

// Waits for the rings of `staging` on every device (all of them if NULL);
// with `release` also destroys their events and forgets them.
hipError_t rings_wait(const void* staging, bool release) {
  std::lock_guard<std::mutex> g(g_rings_m);
  hipError_t first = hipSuccess;
  for (auto it = g_rings.begin(); it != g_rings.end();) {
    if (staging != nullptr && it->first.first != staging) {
      ++it;
      continue;
    }
    const hipError_t e = ring_drain(it->second);
    if (e != hipSuccess && first == hipSuccess) first = e;
    if (!release) {
      ++it;
      continue;
    }
    int prev = -1;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(it->first.second);
    for (int b = 0; b < kMaxSlots; ++b)
      if (it->second->ev[b] != nullptr) (void)hipEventDestroy(it->second->ev[b]);
    if (prev >= 0) (void)hipSetDevice(prev);
    delete it->second;
    it = g_rings.erase(it);
  }
  return first;
}

// Sets the ring's layout, waiting for every slot first if it changes, and
// creates the events it needs (on the current device).
hipError_t ring_layout(Ring* r, int slots, int64_t slot_bytes) {
  if (r->slots != slots || r->slot_bytes != slot_bytes) {
    const hipError_t e = ring_drain(r);
    if (e != hipSuccess) return e;
    r->slots = slots;
    r->slot_bytes = slot_bytes;
    r->next = 0;
  }
  for (int b = 0; b < slots; ++b) {
    if (r->ev[b] != nullptr) continue;
    const hipError_t e = hipEventCreateWithFlags(&r->ev[b], hipEventDisableTiming);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

struct RowCopy {
  const char* name;
  int64_t src, bytes;
  uint8_t* dst;
};

// Copies every range through a ring of pinned staging slots: a slot is
// refilled (pread by the pool) once its previous hipMemcpyAsync has read it,
// so the reads of later slots overlap the PCIe copies of earlier ones.
// Returns after the last copy has completed.
int staged_copy(StFile* f, const RowCopy* copies, int n, void* staging, int64_t staging_bytes, hipStream_t st,
                const char* fn) {
  int64_t total = 0;
  for (int i = 0; i < n; ++i) total += copies[i].bytes;
  if (total == 0) return KLC_OK;
  KLC_REQUIRE(staging != nullptr && staging_bytes >= 2 * 4096, KLC_ERR_ARGUMENT,
              "%s: staging of %lld bytes (at least 8 KiB, two slots)", fn, (long long)staging_bytes);
  int slots = (int)std::min<int64_t>(kMaxSlots, std::max<int64_t>(2, staging_bytes / kCopySlotBytes));
  const int64_t slot = std::min<int64_t>(kCopySlotBytes, staging_bytes / slots / 4096 * 4096);
  // packs of earlier klc_st_load_mxfp4_packed calls may still read the staging
  hipError_t herr = rings_wait(staging, false);
  KLC_REQUIRE(herr == hipSuccess, KLC_ERR_HIP, "%s: %s", fn, hipGetErrorString(herr));
  hipEvent_t* done = nullptr;
  herr = slot_events(slots, &done);
  KLC_REQUIRE(herr == hipSuccess, KLC_ERR_HIP, "%s: %s", fn, hipGetErrorString(herr));
  bool used[kMaxSlots] = {};
  int rc = KLC_OK;
  int64_t k = 0;  // chunks issued so far
  for (int i = 0; i < n && rc == KLC_OK; ++i) {
    for (int64_t off = 0, len = 0; off < copies[i].bytes && rc == KLC_OK; off += len, ++k) {
      const int b = (int)(k % slots);
      // the first chunk is a quarter slot: the first copy starts sooner
      const int64_t cap = k == 0 ? std::max<int64_t>(4096, slot / 4 / 4096 * 4096) : slot;
      len = std::min<int64_t>(cap, copies[i].bytes - off);
      uint8_t* buf = static_cast<uint8_t*>(staging) + b * slot;
      if (used[b] && (herr = hipEventSynchronize(done[b])) != hipSuccess) {
        rc = set_error(KLC_ERR_HIP, "%s: %s", fn, hipGetErrorString(herr));
        break;
      }
      const int rerr = parallel_read(f, buf, len, copies[i].src + off);
      if (rerr != 0) {
        rc = set_error(KLC_ERR_ARGUMENT, "%s: read of '%s' failed: %s", fn, copies[i].name, strerror(rerr));
        break;
      }
      herr = hipMemcpyAsync(copies[i].dst + off, buf, (size_t)len, hipMemcpyHostToDevice, st);
      if (herr == hipSuccess) herr = hipEventRecord(done[b], st);
      used[b] = true;
      if (herr != hipSuccess) rc = set_error(KLC_ERR_HIP, "%s: %s", fn, hipGetErrorString(herr));
    }
  }
  // the caller may reuse the staging buffer on return
  for (int b = 0; b < slots; ++b) {
    if (used[b] && (herr = hipEventSynchronize(done[b])) != hipSuccess && rc == KLC_OK)
      rc = set_error(KLC_ERR_HIP, "%s: %s", fn, hipGetErrorString(herr));
  }
  return rc;
}

}  // namespace
}  // namespace klc

extern "C" int klc_st_copy_rows_to_device(void* handle, const char* name, int64_t first, int64_t count,
                                          void* staging, int64_t staging_bytes, void* dst, void* stream) {
  StFile* f = static_cast<StFile*>(handle);
  RowCopy c{name, 0, 0, static_cast<uint8_t*>(dst)};
  const int rc = row_range(f, name, first, count, &c.src, &c.bytes);
  if (rc) return rc;
  KLC_REQUIRE(dst || c.bytes == 0, KLC_ERR_ARGUMENT, "klc_st_copy_rows_to_device: null destination");
  return staged_copy(f, &c, 1, staging, staging_bytes, as_stream(stream), "klc_st_copy_rows_to_device");
}

extern "C" int klc_st_copy_rows_batch(void* handle, int n, const char* const* names, const int64_t* firsts,
                                      const int64_t* counts, void* const* dsts, void* staging, int64_t staging_bytes,
                                      void* stream) {
  StFile* f = static_cast<StFile*>(handle);
  KLC_REQUIRE(n >= 0 && (n == 0 || (names && firsts && counts && dsts)), KLC_ERR_ARGUMENT,
              "klc_st_copy_rows_batch: null arrays or negative count");
  std::vector<RowCopy> copies((size_t)n);
  for (int i = 0; i < n; ++i) {
    copies[i].name = names[i];
    copies[i].dst = static_cast<uint8_t*>(dsts[i]);
    const int rc = row_range(f, names[i], firsts[i], counts[i], &copies[i].src, &copies[i].bytes);
    if (rc) return rc;
    KLC_REQUIRE(dsts[i] || copies[i].bytes == 0, KLC_ERR_ARGUMENT, "klc_st_copy_rows_batch: null destination %d",
                i);
  }
  return staged_copy(f, copies.data(), n, staging, staging_bytes, as_stream(stream), "klc_st_copy_rows_batch");
}

extern "C" int klc_st_load_mxfp4_packed(void* handle, const char* blocks_name, const char* scales_name,
                                        int64_t expert, void* staging, int64_t staging_bytes, void* packed,
                                        void* stream) {
  StFile* f = static_cast<StFile*>(handle);
  KLC_REQUIRE(f && blocks_name && scales_name && packed, KLC_ERR_ARGUMENT, "klc_st_load_mxfp4_packed: null argument");
  const auto bi = f->tensors.find(blocks_name);
  const auto si = f->tensors.find(scales_name);
  KLC_REQUIRE(bi != f->tensors.end(), KLC_ERR_ARGUMENT, "safetensors: no tensor named '%s'", blocks_name);
  KLC_REQUIRE(si != f->tensors.end(), KLC_ERR_ARGUMENT, "safetensors: no tensor named '%s'", scales_name);
  const StTensor& bt = bi->second;
  const StTensor& sc = si->second;
  KLC_REQUIRE(bt.dtype == "U8" && sc.dtype == "U8" && bt.shape.size() == 4 && sc.shape.size() == 3 &&
                  bt.shape[3] == 16 && bt.shape[0] == sc.shape[0] && bt.shape[1] == sc.shape[1] &&
                  bt.shape[2] == sc.shape[2],
              KLC_ERR_SHAPE,
              "klc_st_load_mxfp4_packed: '%s' / '%s' are not U8 MXFP4 blocks [E, rows, G, 16] and scales [E, rows, G]",
              blocks_name, scales_name);
  const int64_t experts = bt.shape[0], rows = bt.shape[1], groups = bt.shape[2];
  KLC_REQUIRE(expert >= 0 && expert < experts, KLC_ERR_SHAPE, "klc_st_load_mxfp4_packed: expert %lld of %lld",
              (long long)expert, (long long)experts);
  KLC_REQUIRE(rows > 0 && rows % kTileRows == 0 && groups > 0, KLC_ERR_SHAPE,
              "klc_st_load_mxfp4_packed: rows=%lld (a positive multiple of %d) groups=%lld", (long long)rows,
              kTileRows, (long long)groups);
  KLC_REQUIRE(rows < (1 << 30) && groups < (1 << 24), KLC_ERR_UNSUPPORTED, "klc_st_load_mxfp4_packed: matrix too large");
  // one 64-row tile's checkpoint bytes: blocks then scales
  const int64_t tile_blocks = kTileRows * groups * 16, tile_scales = kTileRows * groups;
  const int64_t tile_bytes = tile_blocks + tile_scales;
  KLC_REQUIRE(((uintptr_t)staging | (uintptr_t)packed) % 16 == 0, KLC_ERR_ARGUMENT,
              "klc_st_load_mxfp4_packed: staging and packed must be 16-byte aligned");
  KLC_REQUIRE(staging && staging_bytes >= 2 * tile_bytes, KLC_ERR_ARGUMENT,
              "klc_st_load_mxfp4_packed: staging of %lld bytes (two slots of at least one tile, %lld bytes, each)",
              (long long)staging_bytes, (long long)tile_bytes);
  // slots of whole tiles, at most kSlotBytes unless one tile is larger
  const int64_t unit = std::max(kSlotBytes, tile_bytes);
  const int slots = (int)std::min<int64_t>(kMaxSlots, std::max<int64_t>(2, staging_bytes / unit));
  const int64_t slot_tiles = std::max<int64_t>(1, std::min(kSlotBytes, staging_bytes / slots) / tile_bytes);
  const int64_t slot_bytes = slot_tiles * tile_bytes;
  KLC_REQUIRE(slots * slot_bytes <= staging_bytes, KLC_ERR_ARGUMENT,
              "klc_st_load_mxfp4_packed: %d slots of %lld bytes exceed the staging", slots, (long long)slot_bytes);
  const int64_t tiles = rows / kTileRows;
  const int64_t blocks_src = f->data_start + bt.begin + expert * rows * groups * 16;
  const int64_t scales_src = f->data_start + sc.begin + expert * rows * groups;
  uint8_t* out_blocks = static_cast<uint8_t*>(packed);
  uint8_t* out_scales = out_blocks + packed_block_bytes(rows, groups);
  const int64_t scale_tile_bytes = (int64_t)kTileRows * 4 * packed_scale_record(groups);
  // the pack kernel reads the staging over PCIe: it must be pinned, mapped memory
  void* staging_dev = nullptr;
  hipError_t herr = hipHostGetDevicePointer(&staging_dev, staging, 0);
  if (herr != hipSuccess || staging_dev == nullptr) {
    (void)hipGetLastError();  // handled here: a later launch check must not see it
    return set_error(KLC_ERR_ARGUMENT, "klc_st_load_mxfp4_packed: staging is not pinned host memory (%s)",
                     hipGetErrorString(herr));
  }
  hipStream_t st = as_stream(stream);
  int device = 0;
  herr = hipGetDevice(&device);
  KLC_REQUIRE(herr == hipSuccess, KLC_ERR_HIP, "klc_st_load_mxfp4_packed: %s", hipGetErrorString(herr));
  Ring* ring = ring_of(staging, device);
  herr = ring_layout(ring, slots, slot_bytes);
  KLC_REQUIRE(herr == hipSuccess, KLC_ERR_HIP, "klc_st_load_mxfp4_packed: %s", hipGetErrorString(herr));
  bool idle = true;
  for (int b = 0; b < slots; ++b) idle = idle && !ring->used[b];
  int rc = KLC_OK;
  for (int64_t t0 = 0, nt = 0, k = 0; t0 < tiles && rc == KLC_OK; t0 += nt, ++k) {
    const int b = ring->next;
    ring->next = (b + 1) % slots;
    // with the ring idle, the first chunk is a quarter slot: the GPU starts sooner
    nt = std::min(k == 0 && idle ? std::max<int64_t>(1, slot_tiles / 4) : slot_tiles, tiles - t0);
    const int64_t nb = nt * tile_blocks, ns = nt * tile_scales;
    uint8_t* host = static_cast<uint8_t*>(staging) + b * slot_bytes;
    const uint8_t* mapped = static_cast<const uint8_t*>(staging_dev) + b * slot_bytes;
    // the slot's previous pack (of this call or an earlier one) has read it
    if (ring->used[b]) {
      herr = hipEventSynchronize(ring->ev[b]);
      ring->used[b] = false;
      if (herr != hipSuccess) {
        rc = set_error(KLC_ERR_HIP, "klc_st_load_mxfp4_packed: %s", hipGetErrorString(herr));
        break;
      }
    }
    int rerr = parallel_read(f, host, nb, blocks_src + t0 * tile_blocks);
    if (rerr == 0) rerr = parallel_read(f, host + nb, ns, scales_src + t0 * tile_scales);
    if (rerr != 0) {
      rc = set_error(KLC_ERR_ARGUMENT, "klc_st_load_mxfp4_packed: read of '%s' failed: %s", blocks_name,
                     strerror(rerr));
      break;
    }
    rc = launch_pack_from_host(mapped, mapped + nb, out_blocks + t0 * groups * 1024, out_scales + t0 * scale_tile_bytes,
                               (int)(nt * kTileRows), (int)groups, st);
    if (rc != KLC_OK) break;
    herr = hipEventRecord(ring->ev[b], st);
    if (herr != hipSuccess) {
      rc = set_error(KLC_ERR_HIP, "klc_st_load_mxfp4_packed: %s", hipGetErrorString(herr));
      break;
    }
    ring->used[b] = true;
  }
  if (rc != KLC_OK) {  // no pack may still read the staging
    (void)hipStreamSynchronize(st);
    (void)ring_drain(ring);
  }
  return rc;
}

extern "C" int klc_st_staging_wait(const void* staging) {
  KLC_REQUIRE(staging, KLC_ERR_ARGUMENT, "klc_st_staging_wait: null staging");
  const hipError_t e = rings_wait(staging, false);
  KLC_REQUIRE(e == hipSuccess, KLC_ERR_HIP, "klc_st_staging_wait: %s", hipGetErrorString(e));
  return KLC_OK;
}

extern "C" int klc_st_staging_release(const void* staging) {
  KLC_REQUIRE(staging, KLC_ERR_ARGUMENT, "klc_st_staging_release: null staging");
  const hipError_t e = rings_wait(staging, true);
  KLC_REQUIRE(e == hipSuccess, KLC_ERR_HIP, "klc_st_staging_release: %s", hipGetErrorString(e));
  return KLC_OK;
}
