// Device state, failure handling, the host-range registry, host staging, copies and graph capture.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <cerrno>
#include <map>
#include <mutex>
#include <vector>

#include <fcntl.h>
#include <sys/ioctl.h>
#include <unistd.h>

#include "common.h"

namespace llhip {

// ---- failure ----------------------------------------------------------------------------------------------------

namespace {
std::mutex fail_mutex;
LlhipFailFn fail_handler = nullptr;
int fail_mode = LLHIP_FAIL_EXIT;
char last_error[512] = "";
} // namespace

// ---- HBM budget (src/loader.c:28-56) --------------------------------------------------------------------------------
//
// Every device allocation the library makes or hands out (registered weights, llhip_malloc buffers such as the K/V
// caches, aligned BF16 panels, the staging arena, the attention and split-K workspaces) is claimed against
// LLAMA_HBM_BUDGET_GIB, by default the device's whole memory; a claim beyond it fails with the reference's message.
namespace {
std::mutex budget_mutex;
size_t hbm_claimed = 0;
size_t device_total = 0; // the device's memory, known once it is open
} // namespace

// The budget in bytes, or 0 after raise for a malformed LLAMA_HBM_BUDGET_GIB (parsed on every claim, like the
// reference, so a bad value never goes unnoticed).
static size_t budget_bytes() {
  const char *value = getenv("LLAMA_HBM_BUDGET_GIB");
  if (!value || !*value)
    return device_total;
  char *end;
  const double gib = strtod(value, &end);
  if (*end || !(gib > 0) || gib > (double)(1 << 20))
    return raise("LLAMA_HBM_BUDGET_GIB must be a positive number of GiB"), 0;
  return (size_t)(gib * (double)(1 << 30));
}

bool hbm_claim(size_t bytes, const char *what) {
  const size_t budget = budget_bytes();
  if (!budget)
    return false;
  size_t left;
  {
    std::lock_guard<std::mutex> lock(budget_mutex);
    if (bytes <= budget && hbm_claimed <= budget - bytes) {
      hbm_claimed += bytes;
      return true;
    }
    left = budget > hbm_claimed ? budget - hbm_claimed : 0;
  }
  return raise("%s need %zu bytes of HBM but LLAMA_HBM_BUDGET_GIB leaves %zu of %zu", what, bytes, left, budget);
}

void hbm_release(size_t bytes) {
  std::lock_guard<std::mutex> lock(budget_mutex);
  hbm_claimed -= bytes < hbm_claimed ? bytes : hbm_claimed;
}

bool raise(const char *format, ...) {
  char message[512];
  va_list args;
  va_start(args, format);
  vsnprintf(message, sizeof(message), format, args);
  va_end(args);
  std::lock_guard<std::mutex> lock(fail_mutex);
  snprintf(last_error, sizeof(last_error), "%s", message);
  if (fail_mode == LLHIP_FAIL_RECORD)
    return false;
  if (fail_handler)
    fail_handler(message);
  fprintf(stderr, "error: %s\n", message);
  fflush(stderr);
  exit(EXIT_FAILURE);
}

bool check_hip(hipError_t status, const char *what) {
  if (status == hipSuccess)
    return true;
  return raise("HIP call %s failed: %s", what, hipGetErrorString(status));
}

// ---- device -------------------------------------------------------------------------------------------------------

namespace {
std::mutex device_mutex;
Device the_device;
char device_name[256] = "";
} // namespace

Device &device() { return the_device; }

bool ensure_device() {
  if (the_device.ready)
    return true;
  std::lock_guard<std::mutex> lock(device_mutex);
  if (the_device.ready)
    return true;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
    (void)hipGetLastError();
    return raise("no HIP device is available (this library runs the matmul hot path on an MI355X)");
  }
  int ordinal = 0;
  if (const char *env = getenv("LLAMA_HIP_DEVICE"); env && *env) {
    char *end;
    long value = strtol(env, &end, 10);
    if (*end || value < 0 || value >= count)
      return raise("LLAMA_HIP_DEVICE must be an integer in 0..%d", count - 1);
    ordinal = (int)value;
  }
  if (!LLHIP_CHECK(hipSetDevice(ordinal)))
    return false;
  hipDeviceProp_t props;
  if (!LLHIP_CHECK(hipGetDeviceProperties(&props, ordinal)))
    return false;
  if (strncmp(props.gcnArchName, "gfx950", 6) != 0)
    return raise("device %d is %s; this library is built for gfx950 (MI355X)", ordinal, props.gcnArchName);
  snprintf(device_name, sizeof(device_name), "%s%s%s, %d CUs", props.name, props.name[0] ? " " : "",
           props.gcnArchName, props.multiProcessorCount);
  hipStream_t stream;
  if (!LLHIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking)))
    return false;
  device_total = props.totalGlobalMem;
  if (!hbm_claim((size_t)LLHIP_SPLIT_SLOTS * (256 * 128 * sizeof(float) + sizeof(unsigned)) + 64,
                 "the split-K workspace"))
    return false;
  int *flags, *host_flags;
  if (!LLHIP_CHECK(hipMalloc(&flags, 64)) || !LLHIP_CHECK(hipHostMalloc((void **)&host_flags, 64, hipHostMallocDefault)))
    return false;
  int zero[16] = {0};
  if (!LLHIP_CHECK(hipMemcpy(flags, zero, sizeof(zero), hipMemcpyHostToDevice)))
    return false;
  void *partial;
  unsigned *arrivals;
  if (!LLHIP_CHECK(hipMalloc(&partial, (size_t)LLHIP_SPLIT_SLOTS * 256 * 128 * sizeof(float))) ||
      !LLHIP_CHECK(hipMalloc((void **)&arrivals, LLHIP_SPLIT_SLOTS * sizeof(unsigned))) ||
      !LLHIP_CHECK(hipMemset(arrivals, 0, LLHIP_SPLIT_SLOTS * sizeof(unsigned))))
    return false;
  if (!attention_scratch_setup(ordinal)) // the allocation-free attention's array: its address on this device
    return false;
  the_device.split_partial = partial;
  the_device.split_count = arrivals;
  the_device.ordinal = ordinal;
  the_device.stream = stream;
  the_device.error_flags = flags;
  the_device.host_flags = host_flags;
  the_device.cu_count = props.multiProcessorCount;
  the_device.ready = true;
  return true;
}

// A device error flag set since the last check becomes the failure of this call (the flags then cleared).
bool report_flags(const int *flags) {
  Device &dev = the_device;
  if (flags[0] || flags[1] || flags[2]) {
    int zero[16] = {0};
    (void)hipMemcpy(dev.error_flags, zero, sizeof(zero), hipMemcpyHostToDevice);
    return raise(flags[0]   ? "nonfinite activation during INT8 quantization"
                 : flags[1] ? "nonfinite value in softmax"
                            : "embedding row id outside the table");
  }
  return true;
}

bool synchronize_and_check() {
  if (!ensure_device())
    return false;
  Device &dev = the_device;
  if (dev.capturing)
    return raise("a host-visible wait was requested during graph capture");
  if (!flush_pending_quantize())
    return false;
  // the flags come back behind the stream's work, so one wait covers both (a blocking copy after the wait would be a
  // second round trip to the device)
  if (!LLHIP_CHECK(hipMemcpyAsync(dev.host_flags, dev.error_flags, 16 * sizeof(int), hipMemcpyDeviceToHost,
                                  dev.stream)) ||
      !LLHIP_CHECK(hipStreamSynchronize(dev.stream)))
    return false;
  int flags[16];
  memcpy(flags, dev.host_flags, sizeof(flags));
  return report_flags(flags);
}

// ---- registry of uploaded host ranges ----------------------------------------------------------------------------

namespace {
// A mapped segment of a file registered on its own (LLAMA_HIP_REGISTER_MAPPINGS): its address range and what it
// maps, the file (device and inode) and the file offset at its start.
struct Segment {
  uintptr_t start, end;
  unsigned long long offset, ino;
  unsigned dev_major, dev_minor;
};
struct Region {
  size_t bytes;
  void *device;
  std::vector<Segment> segments; // empty for llhip_register_host's ranges
};
std::mutex registry_mutex;
std::map<uintptr_t, Region> registry;
std::map<void *, size_t> allocations; // llhip_malloc's buffers and their claimed bytes (under registry_mutex)

// The device copy of p when p lies inside a registered range, else nullptr; *room receives the bytes of the range
// from p to its end, *start the range's start and *automatic whether it was registered as a file mapping.
void *lookup(const void *p, size_t *room = nullptr, uintptr_t *start = nullptr, bool *automatic = nullptr) {
  std::lock_guard<std::mutex> lock(registry_mutex);
  if (registry.empty())
    return nullptr;
  uintptr_t addr = (uintptr_t)p;
  auto it = registry.upper_bound(addr);
  if (it == registry.begin())
    return nullptr;
  --it;
  if (addr >= it->first + it->second.bytes)
    return nullptr;
  if (room)
    *room = it->first + it->second.bytes - addr;
  if (start)
    *start = it->first;
  if (automatic)
    *automatic = !it->second.segments.empty();
  return (char *)it->second.device + (addr - it->first);
}

// 1: device memory with at least `bytes` from p to the end of its allocation; -1: device memory that is shorter
// (the launch would read or write past it); 0: not device memory.
int device_extent(const void *p, size_t bytes) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (attr.type != hipMemoryTypeDevice)
    return 0;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
    (void)hipGetLastError();
    return 1; // device memory whose extent the runtime cannot tell: trusted, like any C caller's buffer
  }
  return (uintptr_t)p + bytes <= (uintptr_t)base + size ? 1 : -1;
}

// LLAMA_HIP_REGISTER_MAPPINGS=1 (read once): a host input that lies in a read-only mapping of a regular file, a file
// no executable segment maps (so not a program or a library), is registered whole on its first use: uploaded to HBM
// once, and resolved to that copy by every later call. An unchanged caller that takes its weight views from a mapped
// checkpoint (the reference maps it read-only, src/runtime.c:306, and views its tensors in place, src/tp.c:897-903)
// then runs on resident weights instead of staging them over PCIe per call.
bool register_mappings_enabled() {
  static const bool on = [] {
    const char *v = getenv("LLAMA_HIP_REGISTER_MAPPINGS");
    return v && !strcmp(v, "1");
  }();
  return on;
}

struct MapEntry {
  uintptr_t start, end;
  unsigned long long offset, inode;
  unsigned dev_major, dev_minor;
  bool read, write, exec, file;
};

std::vector<MapEntry> read_maps() {
  std::vector<MapEntry> out;
  FILE *f = fopen("/proc/self/maps", "r");
  if (!f)
    return out;
  char line[4096];
  while (fgets(line, sizeof(line), f)) {
    MapEntry m{};
    char perms[8] = {0};
    int used = 0;
    unsigned long start, end;
    if (sscanf(line, "%lx-%lx %7s %llx %x:%x %llu %n", &start, &end, perms, &m.offset, &m.dev_major, &m.dev_minor,
               &m.inode, &used) < 7)
      continue;
    m.start = start;
    m.end = end;
    m.read = perms[0] == 'r';
    m.write = perms[1] == 'w';
    m.exec = perms[2] == 'x';
    m.file = m.inode != 0 && line[used] == '/';
    out.push_back(m);
  }
  fclose(f);
  return out;
}

// The mapping that covers address a now. PROCMAP_QUERY (an ioctl on /proc/self/maps, Linux 6.11 and later; its
// structure is the kernel's uapi one) asks for that one mapping directly; where the kernel lacks it, the whole table
// is read.
struct ProcmapQuery {
  uint64_t size, query_flags, query_addr, vma_start, vma_end, vma_flags, vma_page_size, vma_offset, inode;
  uint32_t dev_major, dev_minor, vma_name_size, build_id_size;
  uint64_t vma_name_addr, build_id_addr;
};
const unsigned long kProcmapQuery = _IOWR('f', 17, ProcmapQuery);
constexpr uint64_t kVmaReadable = 1, kVmaWritable = 2, kVmaExecutable = 4;

bool vma_at(uintptr_t a, MapEntry *out) {
  // kept open for the process; a forked child, whose inherited descriptor would show the parent's table, opens its own
  static std::mutex fd_mutex;
  static int fd = -1;
  static pid_t owner = 0;
  static std::atomic<bool> no_query{false};
  int qfd;
  {
    std::lock_guard<std::mutex> lock(fd_mutex);
    if (owner != getpid()) {
      if (fd >= 0)
        close(fd);
      fd = open("/proc/self/maps", O_RDONLY | O_CLOEXEC);
      owner = getpid();
    }
    qfd = fd;
  }
  if (qfd >= 0 && !no_query.load()) {
    ProcmapQuery q{};
    q.size = sizeof(q);
    q.query_addr = a;
    if (ioctl(qfd, kProcmapQuery, &q) == 0) {
      *out = MapEntry{(uintptr_t)q.vma_start, (uintptr_t)q.vma_end, q.vma_offset, q.inode, q.dev_major, q.dev_minor,
                      (q.vma_flags & kVmaReadable) != 0, (q.vma_flags & kVmaWritable) != 0,
                      (q.vma_flags & kVmaExecutable) != 0, q.inode != 0};
      return true;
    }
    if (errno == ENOENT)
      return false; // nothing is mapped there
    no_query.store(true); // an older kernel: ENOTTY or EINVAL
  }
  for (const MapEntry &m : read_maps())
    if (a >= m.start && a < m.end) {
      *out = m;
      return true;
    }
  return false;
}

std::mutex mapping_mutex;
std::vector<std::pair<uintptr_t, uintptr_t>> mappings_declined; // ranges already found not to qualify
int register_range(const void *host, size_t bytes, std::vector<Segment> segments);

// Registers the file mapping around host address p when it qualifies; false otherwise (p then stays staged).
bool register_file_mapping(const void *p) {
  const uintptr_t a = (uintptr_t)p;
  std::lock_guard<std::mutex> lock(mapping_mutex);
  for (const auto &r : mappings_declined)
    if (a >= r.first && a < r.second)
      return false;
  if (lookup(p)) // registered meanwhile by another thread
    return true;
  const std::vector<MapEntry> maps = read_maps();
  size_t i = 0;
  while (i < maps.size() && !(a >= maps[i].start && a < maps[i].end))
    i++;
  if (i == maps.size())
    return false;
  const MapEntry &m = maps[i];
  bool ok = m.file && m.read && !m.write;
  for (const MapEntry &o : maps) // a program or a library: some segment of the same file is executable
    if (o.exec && o.inode == m.inode && o.dev_major == m.dev_major && o.dev_minor == m.dev_minor)
      ok = false;
  if (!ok) {
    if (mappings_declined.size() < 64)
      mappings_declined.emplace_back(m.start, m.end);
    return false;
  }
  // the whole mapping: neighbouring entries of the same file with continuing offsets and the same permissions
  auto same = [&](const MapEntry &x, const MapEntry &y) {
    return x.inode == y.inode && x.dev_major == y.dev_major && x.dev_minor == y.dev_minor && x.read == y.read &&
           x.write == y.write && x.exec == y.exec && x.end == y.start && x.offset + (y.start - x.start) == y.offset;
  };
  size_t lo = i, hi = i;
  while (lo > 0 && same(maps[lo - 1], maps[lo]))
    lo--;
  while (hi + 1 < maps.size() && same(maps[hi], maps[hi + 1]))
    hi++;
  // what each segment maps, checked again by every later call that resolves into the range (mapping_current)
  std::vector<Segment> segments;
  for (size_t j = lo; j <= hi; j++)
    segments.push_back(Segment{maps[j].start, maps[j].end, maps[j].offset, maps[j].inode, maps[j].dev_major,
                               maps[j].dev_minor});
  return register_range((const void *)maps[lo].start, maps[hi].end - maps[lo].start, std::move(segments)) == 0;
}

// Whether the file mapping registered at `start` still maps, at p, the same place of the same file, read-only: false
// once the caller has unmapped it (and perhaps mapped something else at the same addresses).
bool mapping_current(uintptr_t start, const void *p) {
  const uintptr_t a = (uintptr_t)p;
  Segment seg{};
  {
    std::lock_guard<std::mutex> lock(registry_mutex);
    auto it = registry.find(start);
    if (it == registry.end())
      return false;
    bool found = false;
    for (const Segment &g : it->second.segments)
      if (a >= g.start && a < g.end) {
        seg = g;
        found = true;
        break;
      }
    if (!found)
      return false;
  }
  MapEntry now{};
  return vma_at(a, &now) && now.file && now.read && !now.write && now.inode == seg.ino &&
         now.dev_major == seg.dev_major && now.dev_minor == seg.dev_minor &&
         now.offset + (a - now.start) == seg.offset + (a - seg.start);
}

// Drops the file mapping registered at `start` (its device copy freed once the stream's work is done): the caller
// unmapped it, so a later call with addresses inside it means whatever is mapped there now. False after raise (under
// graph capture, where the stream cannot wait).
bool retire_mapping(uintptr_t start) {
  std::lock_guard<std::mutex> lock(mapping_mutex);
  if (the_device.capturing)
    return raise("a registered file mapping was unmapped or replaced during graph capture");
  size_t bytes = 0;
  {
    std::lock_guard<std::mutex> rl(registry_mutex);
    auto it = registry.find(start);
    if (it == registry.end() || it->second.segments.empty())
      return true; // retired meanwhile by another call
    bytes = it->second.bytes;
  }
  mappings_declined.erase(std::remove_if(mappings_declined.begin(), mappings_declined.end(),
                                         [&](const std::pair<uintptr_t, uintptr_t> &r) {
                                           return r.first < start + bytes && start < r.second;
                                         }),
                          mappings_declined.end());
  return llhip_unregister_host((const void *)start) == 0;
}

// The staging arena for host buffers: grown on demand, reused by every staged call. Calls that stage at most
// kBounceMax bytes copy through a pinned host twin of the arena (the caller's bytes are memcpy'd into it, then one DMA
// per buffer), and read the device error flags back through pinned memory in the same wait, where pageable copies
// take the runtime's slower staging and the flags a second synchronous copy.
void *arena = nullptr;
size_t arena_bytes = 0;
std::mutex arena_mutex;
constexpr size_t kBounceMax = 64u << 20;
void *bounce = nullptr;
size_t bounce_bytes = 0;
int *bounce_flags = nullptr; // 16 ints

bool bounce_room(size_t bytes) {
  if (!bounce_flags) {
    if (hipHostMalloc((void **)&bounce_flags, 16 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      bounce_flags = nullptr;
      return false;
    }
  }
  if (bytes <= bounce_bytes)
    return true;
  if (bounce)
    (void)hipHostFree(bounce);
  bounce = nullptr;
  bounce_bytes = 0;
  const size_t want = std::min(kBounceMax, bytes + (bytes >> 2) + 4096);
  if (hipHostMalloc(&bounce, want, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    bounce = nullptr;
    return false;
  }
  bounce_bytes = want;
  return true;
}
} // namespace

// ---- Call ---------------------------------------------------------------------------------------------------------

// ---- deferred quantization ---------------------------------------------------------------------------------------

namespace {
std::mutex pending_mutex;
bool pending_active = false;
PendingQuantize pending_job;
bool norm_active = false; // a recorded k_rmsnorm (at most one of it and pending_job unconsumed: each flushes the other)
PendingNorm norm_job;
bool rope_active = false; // a recorded k_rope_apply with its cache stores (likewise exclusive of the two above)
PendingRope rope_job;

bool launch_rope_and_stores(const PendingRope &r, hipStream_t stream) {
  if (!launch_rope(r.q, (size_t)r.n_heads * r.head_dim, r.k, (size_t)r.n_kv_heads * r.head_dim, r.table,
                   2 * (size_t)r.head_dim, 1, r.n_heads, r.n_kv_heads, r.head_dim, stream))
    return false;
  for (int i = 0; i < r.stores; i++) {
    const PendingKvStore &st = r.store[i];
    if (!launch_kv_store(st.cache, st.src, (size_t)r.n_kv_heads * r.head_dim, st.pos, 1, r.n_kv_heads, r.head_dim,
                         st.pos_stride, st.head_base, stream))
      return false;
  }
  return true;
}
} // namespace

bool quantize_fusion_enabled() {
  static const bool on = [] {
    const char *env = getenv("LLAMA_HIP_FUSE_QUANT");
    return !(env && !strcmp(env, "0"));
  }();
  return on;
}

void defer_norm(const PendingNorm &job) {
  flush_pending_quantize(); // what was recorded earlier runs first
  std::lock_guard<std::mutex> lock(pending_mutex);
  norm_job = job;
  norm_active = true;
}

void defer_quantize(const PendingQuantize &recorded) {
  PendingQuantize job = recorded;
  {
    // the quantization of a recorded norm's whole output takes the norm along: the GEMV normalizes in its prologue
    std::lock_guard<std::mutex> lock(pending_mutex);
    if (norm_active && norm_job.out == job.x && norm_job.size == job.n && !job.norm_w) {
      job.x = norm_job.x;
      job.norm_w = norm_job.w;
      job.norm_out = norm_job.out;
      job.norm_eps = norm_job.eps;
      norm_active = false;
    }
  }
  flush_pending_quantize();
  std::lock_guard<std::mutex> lock(pending_mutex);
  pending_job = job;
  pending_active = true;
}

bool launch_pending_quantize(const PendingQuantize &job, hipStream_t stream) {
  const float *x = job.x;
  if (job.norm_w) {
    if (!launch_rmsnorm(job.norm_out, job.x, job.norm_w, 1, job.n, job.norm_eps, stream))
      return false;
    x = job.norm_out;
  }
  return launch_quantize(QuantizeJob{job.q, job.s, x, (size_t)job.n, 1, job.n, job.gs}, stream);
}

bool take_pending_quantize(const int8_t *q, const float *s, int n, int gs, PendingQuantize *out) {
  std::lock_guard<std::mutex> lock(pending_mutex);
  if (!pending_active || pending_job.q != q || pending_job.s != s || pending_job.n != n || pending_job.gs != gs)
    return false;
  *out = pending_job;
  pending_active = false;
  return true;
}

bool flush_pending_quantize() {
  PendingQuantize job;
  PendingNorm norm;
  PendingRope rope;
  bool have_job, have_norm, have_rope;
  {
    std::lock_guard<std::mutex> lock(pending_mutex);
    have_job = pending_active;
    have_norm = norm_active;
    have_rope = rope_active;
    job = pending_job;
    norm = norm_job;
    rope = rope_job;
    pending_active = norm_active = rope_active = false;
  }
  if (have_rope && !launch_rope_and_stores(rope, the_device.stream))
    return false;
  if (have_norm && !launch_rmsnorm(norm.out, norm.x, norm.w, 1, norm.size, norm.eps, the_device.stream))
    return false;
  return !have_job || launch_pending_quantize(job, the_device.stream);
}

void defer_rope(const PendingRope &job) {
  flush_pending_quantize(); // what was recorded earlier runs first
  std::lock_guard<std::mutex> lock(pending_mutex);
  rope_job = job;
  rope_job.stores = 0;
  rope_active = true;
}

bool attach_kv_store(const PendingKvStore &store, int n_kv_heads, int head_dim) {
  std::lock_guard<std::mutex> lock(pending_mutex);
  if (!rope_active || rope_job.n_kv_heads != n_kv_heads || rope_job.head_dim != head_dim || rope_job.stores == 2)
    return false;
  // the first store must be of the rotated k, the second of another row (v) at the same position and layout
  if (rope_job.stores == 0 ? store.src != rope_job.k
                           : (store.src == rope_job.k || store.pos != rope_job.store[0].pos ||
                              store.pos_stride != rope_job.store[0].pos_stride ||
                              store.head_base != rope_job.store[0].head_base || store.cache == rope_job.store[0].cache))
    return false;
  rope_job.store[rope_job.stores++] = store;
  return true;
}

bool take_pending_rope(const float *q, const float *key_cache, const float *value_cache, int position,
                       size_t pos_stride, size_t head_base, int n_heads, int n_kv_heads, int head_dim, PendingRope *out) {
  std::lock_guard<std::mutex> lock(pending_mutex);
  const PendingRope &r = rope_job;
  if (!rope_active || r.stores != 2 || r.q != q || r.n_heads != n_heads || r.n_kv_heads != n_kv_heads ||
      r.head_dim != head_dim || r.store[0].cache != key_cache || r.store[1].cache != value_cache ||
      r.store[0].pos != position || r.store[0].pos_stride != pos_stride || r.store[0].head_base != head_base ||
      ((uintptr_t)r.store[1].src & 15) != 0) // the fused kernel reads the new v row as 16-byte vectors
    return false;
  *out = r;
  rope_active = false;
  return true;
}

Call::Call(const char *name, bool keep_pending) : name_(name) {
  if (!ensure_device())
    failed_ = true;
  else if (!keep_pending && !flush_pending_quantize())
    failed_ = true;
}

Call::~Call() {
  if (staged_)
    arena_mutex.unlock();
}

hipStream_t Call::stream() const { return the_device.stream; }

Ref Call::stage(void *host, size_t row_bytes, size_t pitch, size_t rows, bool to_device, bool to_host) {
  if (ncopies_ == (int)(sizeof(copies_) / sizeof(copies_[0]))) {
    failed_ = true;
    raise("%s: too many host buffers in one call", name_);
    return Ref{};
  }
  if (the_device.capturing) {
    failed_ = true;
    raise("%s: host memory cannot be staged during graph capture (register it or pass device memory)", name_);
    return Ref{};
  }
  if (!staged_) {
    arena_mutex.lock(); // one staged call at a time: they share the arena
    staged_ = true;
  }
  size_t bytes = rows ? (rows - 1) * pitch + row_bytes : 0;
  size_t offset = (arena_used_ + 255) & ~(size_t)255;
  arena_used_ = offset + bytes;
  copies_[ncopies_] = Copy{host, offset, row_bytes, pitch, rows, to_device, to_host};
  return Ref{nullptr, ncopies_++};
}

bool plain_host_memory(const void *p, size_t bytes) { return !lookup(p) && device_extent(p, bytes) == 0; }

void *Call::address(const Ref &r) const {
  return r.staged < 0 ? r.direct : (void *)((char *)arena + copies_[r.staged].offset);
}

// lookup(p), with a range registered as a file mapping checked once per call against what is mapped there now: a
// stale range (the caller unmapped it) is retired first, so p resolves to nothing and takes the unregistered route.
void *Call::resolve_registered(const void *p, size_t *room) {
  uintptr_t start = 0;
  bool automatic = false;
  void *dev = lookup(p, room, &start, &automatic);
  if (!dev || !automatic || start == current_mapping_)
    return dev;
  if (mapping_current(start, p)) {
    current_mapping_ = start;
    return dev;
  }
  if (!retire_mapping(start))
    failed_ = true;
  return nullptr;
}

Ref Call::in2d(const void *p, size_t row_bytes, size_t pitch, size_t rows) {
  if (!p || failed_ || !rows)
    return Ref{const_cast<void *>(p), -1};
  const size_t extent = (rows - 1) * pitch + row_bytes;
  size_t room = 0;
  if (void *dev = resolve_registered(p, &room)) {
    if (room < extent) {
      failed_ = true;
      raise("%s: %zu bytes at %p run past the end of their registered range", name_, extent, p);
      return Ref{};
    }
    return Ref{dev, -1};
  }
  const int where = device_extent(p, extent);
  if (where < 0) {
    failed_ = true;
    raise("%s: %zu bytes at device address %p run past the end of its allocation", name_, extent, p);
    return Ref{};
  }
  if (where > 0)
    return Ref{const_cast<void *>(p), -1};
  if (failed_)
    return Ref{};
  if (register_mappings_enabled() && !the_device.capturing && register_file_mapping(p)) {
    uintptr_t start = 0;
    if (void *dev = lookup(p, &room, &start)) {
      current_mapping_ = start; // registered just now from what is mapped
      if (room >= extent)
        return Ref{dev, -1};
    }
  }
  return stage(const_cast<void *>(p), row_bytes, pitch, rows, true, false);
}

Ref Call::out2d(void *p, size_t row_bytes, size_t pitch, size_t rows, bool read_too) {
  if (!p || failed_ || !rows)
    return Ref{p, -1};
  if (resolve_registered(p)) {
    failed_ = true;
    raise("%s: an output lies inside a registered (read-only) weight range", name_);
    return Ref{};
  }
  const size_t extent = (rows - 1) * pitch + row_bytes;
  const int where = device_extent(p, extent);
  if (where < 0) {
    failed_ = true;
    raise("%s: %zu bytes at device address %p run past the end of its allocation", name_, extent, p);
    return Ref{};
  }
  if (where > 0)
    return Ref{p, -1};
  return stage(p, row_bytes, pitch, rows, read_too, true);
}

bool Call::ready() {
  if (failed_)
    return false;
  if (!staged_)
    return true;
  if (arena_used_ > arena_bytes) {
    if (arena) {
      (void)hipStreamSynchronize(the_device.stream);
      (void)hipFree(arena);
      hbm_release(arena_bytes);
    }
    arena = nullptr;
    arena_bytes = 0;
    size_t want = arena_used_ + (arena_used_ >> 2) + 4096;
    if (!hbm_claim(want, "the staging arena")) {
      failed_ = true;
      return false;
    }
    if (!LLHIP_CHECK(hipMalloc(&arena, want))) {
      hbm_release(want);
      arena = nullptr;
      failed_ = true;
      return false;
    }
    arena_bytes = want;
  }
  bounced_ = arena_used_ <= kBounceMax && bounce_room(arena_used_);
  for (int i = 0; i < ncopies_; i++) {
    Copy &c = copies_[i];
    if (!c.to_device || !c.rows)
      continue;
    bool ok;
    if (bounced_) { // the rows into the pinned twin (the pitch gaps are never read), then one DMA of the extent
      char *b = (char *)bounce + c.offset;
      if (c.pitch == c.row_bytes)
        memcpy(b, c.host, c.row_bytes * c.rows);
      else
        for (size_t r = 0; r < c.rows; r++)
          memcpy(b + r * c.pitch, (const char *)c.host + r * c.pitch, c.row_bytes);
      ok = LLHIP_CHECK(hipMemcpyAsync((char *)arena + c.offset, b, (c.rows - 1) * c.pitch + c.row_bytes,
                                      hipMemcpyHostToDevice, the_device.stream));
    } else {
      ok = LLHIP_CHECK(hipMemcpy2DAsync((char *)arena + c.offset, c.pitch, c.host, c.pitch, c.row_bytes, c.rows,
                                        hipMemcpyHostToDevice, the_device.stream));
    }
    if (!ok) {
      failed_ = true;
      return false;
    }
  }
  return true;
}

bool Call::finish() {
  if (failed_)
    return false;
  if (!staged_)
    return true;
  if (bounced_) { // outputs and the error flags into pinned memory, one wait, then the rows to the caller
    if (!flush_pending_quantize())
      return false;
    for (int i = 0; i < ncopies_; i++) {
      Copy &c = copies_[i];
      if (c.to_host && c.rows &&
          !LLHIP_CHECK(hipMemcpyAsync((char *)bounce + c.offset, (char *)arena + c.offset,
                                      (c.rows - 1) * c.pitch + c.row_bytes, hipMemcpyDeviceToHost, the_device.stream)))
        return false;
    }
    if (!LLHIP_CHECK(hipMemcpyAsync(bounce_flags, the_device.error_flags, 16 * sizeof(int), hipMemcpyDeviceToHost,
                                    the_device.stream)) ||
        !LLHIP_CHECK(hipStreamSynchronize(the_device.stream)))
      return false;
    for (int i = 0; i < ncopies_; i++) {
      Copy &c = copies_[i];
      if (!c.to_host || !c.rows)
        continue;
      const char *b = (const char *)bounce + c.offset;
      if (c.pitch == c.row_bytes)
        memcpy(c.host, b, c.row_bytes * c.rows);
      else
        for (size_t r = 0; r < c.rows; r++)
          memcpy((char *)c.host + r * c.pitch, b + r * c.pitch, c.row_bytes);
    }
    return report_flags(bounce_flags);
  }
  for (int i = 0; i < ncopies_; i++) {
    Copy &c = copies_[i];
    if (!c.to_host || !c.rows)
      continue;
    if (!LLHIP_CHECK(hipMemcpy2DAsync(c.host, c.pitch, (char *)arena + c.offset, c.pitch, c.row_bytes, c.rows,
                                      hipMemcpyDeviceToHost, the_device.stream)))
      return false;
  }
  return synchronize_and_check();
}

namespace {
int register_range(const void *host, size_t bytes, std::vector<Segment> segments) {
  if (!ensure_device())
    return -1;
  if (!host || !bytes)
    return raise("llhip_register_host: empty range"), -1;
  {
    std::lock_guard<std::mutex> lock(registry_mutex);
    uintptr_t a = (uintptr_t)host;
    for (auto &kv : registry)
      if (a < kv.first + kv.second.bytes && kv.first < a + bytes)
        return raise("llhip_register_host: range overlaps a registered range"), -1;
  }
  void *dev;
  if (!hbm_claim(bytes, "registered weights"))
    return -1;
  if (!LLHIP_CHECK(hipMalloc(&dev, bytes)))
    return hbm_release(bytes), -1;
  if (!LLHIP_CHECK(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice))) {
    (void)hipFree(dev);
    hbm_release(bytes);
    return -1;
  }
  std::lock_guard<std::mutex> lock(registry_mutex);
  registry[(uintptr_t)host] = Region{bytes, dev, std::move(segments)};
  return 0;
}
} // namespace

// llhip_register_host: a range with no file identity to check.
int register_range_host(const void *host, size_t bytes) { return register_range(host, bytes, {}); }

} // namespace llhip

// ---- C ABI: device and residency ----------------------------------------------------------------------------------

using namespace llhip;

extern "C" {

int llhip_init(void) { return ensure_device() ? 0 : -1; }

const char *llhip_device_name(void) { return ensure_device() ? device_name : ""; }

int llhip_device_cu_count(void) { return ensure_device() ? the_device.cu_count : 0; }

void *llhip_stream(void) { return ensure_device() ? (void *)the_device.stream : nullptr; }

void llhip_synchronize(void) { (void)synchronize_and_check(); }


int llhip_register_host(const void *host, size_t bytes) { return llhip::register_range_host(host, bytes); }

int llhip_unregister_host(const void *host) {
  if (!ensure_device())
    return -1;
  void *dev = nullptr;
  size_t bytes = 0;
  {
    std::lock_guard<std::mutex> lock(registry_mutex);
    auto it = registry.find((uintptr_t)host);
    if (it == registry.end())
      return raise("llhip_unregister_host: %p is not the start of a registered range", host), -1;
    dev = it->second.device;
    bytes = it->second.bytes;
    registry.erase(it);
  }
  if (!LLHIP_CHECK(hipStreamSynchronize(the_device.stream)))
    return -1;
  hbm_release(bytes);
  return LLHIP_CHECK(hipFree(dev)) ? 0 : -1;
}

void *llhip_resolve(const void *host) { return lookup(host); }

void *llhip_malloc(size_t bytes) {
  if (!ensure_device())
    return nullptr;
  bytes = bytes ? bytes : 1;
  if (!hbm_claim(bytes, "llhip_malloc"))
    return nullptr;
  void *p = nullptr;
  if (!LLHIP_CHECK(hipMalloc(&p, bytes)))
    return hbm_release(bytes), nullptr;
  std::lock_guard<std::mutex> lock(registry_mutex);
  allocations[p] = bytes;
  return p;
}

void llhip_free(void *p) {
  if (!p || !ensure_device() || !flush_pending_quantize())
    return;
  if (!LLHIP_CHECK(hipStreamSynchronize(the_device.stream)))
    return;
  {
    std::lock_guard<std::mutex> lock(registry_mutex);
    auto it = allocations.find(p);
    if (it != allocations.end()) {
      hbm_release(it->second);
      allocations.erase(it);
    }
  }
  (void)LLHIP_CHECK(hipFree(p));
}

size_t placement_hbm_budget(void) {
  if (!device_total && !getenv("LLAMA_HBM_BUDGET_GIB"))
    (void)ensure_device(); // the default is the device's memory
  return budget_bytes();
}

size_t llhip_hbm_claimed(void) {
  std::lock_guard<std::mutex> lock(budget_mutex);
  return hbm_claimed;
}

void llhip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (ensure_device() && flush_pending_quantize() && bytes && LLHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, the_device.stream)))
    (void)LLHIP_CHECK(hipStreamSynchronize(the_device.stream));
}

void llhip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (ensure_device() && flush_pending_quantize() && bytes && LLHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, the_device.stream)))
    (void)LLHIP_CHECK(hipStreamSynchronize(the_device.stream));
}

void llhip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (ensure_device() && flush_pending_quantize() && bytes)
    (void)LLHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, the_device.stream));
}

int llhip_graph_begin(void) {
  if (!ensure_device())
    return -1;
  if (the_device.capturing)
    return raise("llhip_graph_begin: a capture is already open"), -1;
  if (!LLHIP_CHECK(hipStreamBeginCapture(the_device.stream, hipStreamCaptureModeThreadLocal)))
    return -1;
  the_device.capturing = true;
  return 0;
}

void *llhip_graph_end(void) {
  if (!ensure_device() || !the_device.capturing) {
    raise("llhip_graph_end: no capture is open");
    return nullptr;
  }
  const bool flushed = flush_pending_quantize(); // a recorded quantization belongs to the captured sequence
  the_device.capturing = false;
  hipGraph_t graph;
  if (!LLHIP_CHECK(hipStreamEndCapture(the_device.stream, &graph)))
    return nullptr;
  hipGraphExec_t exec;
  bool ok = flushed && LLHIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  (void)hipGraphDestroy(graph);
  return ok ? (void *)exec : nullptr;
}

int llhip_graph_launch(void *graph) {
  if (!ensure_device() || !graph)
    return -1;
  return LLHIP_CHECK(hipGraphLaunch((hipGraphExec_t)graph, the_device.stream)) ? 0 : -1;
}

void llhip_graph_destroy(void *graph) {
  if (graph && ensure_device() && LLHIP_CHECK(hipStreamSynchronize(the_device.stream)))
    (void)hipGraphExecDestroy((hipGraphExec_t)graph);
}

void llhip_set_fail_handler(LlhipFailFn handler) {
  std::lock_guard<std::mutex> lock(fail_mutex);
  fail_handler = handler;
}

void llhip_set_fail_mode(int mode) {
  std::lock_guard<std::mutex> lock(fail_mutex);
  fail_mode = mode == LLHIP_FAIL_RECORD ? LLHIP_FAIL_RECORD : LLHIP_FAIL_EXIT;
}

const char *llhip_last_error(void) { return last_error; }

void llhip_clear_error(void) {
  std::lock_guard<std::mutex> lock(fail_mutex);
  last_error[0] = '\0';
}

} // extern "C"
