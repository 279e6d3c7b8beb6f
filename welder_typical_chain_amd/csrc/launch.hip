// launch.hip -- host side of the launcher C-ABI (include/wtc/wtc_hip.h):
// argument checks, the launch plan, the per-stream default workspaces, the
// host-visible timeout mailbox, the cross-stream ordering of exchange-path
// calls, and the kernel launches for the exchange, split, row-block and
// unfused paths.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "tile_layout.h"
#include "variants.h"
#include "wtc/wtc_hip.h"
#include "wtc_kernels.h"

namespace wtc {
// Waves of rescale_rows_kernel per row: enough for 16 waves per CU when rows
// are few (wide rows), at most 8.
int rescale_waves_per_row(int64_t rows_total, int cu_count) {
  int wpr = 1;
  while (wpr < 8 && rows_total * wpr < 16ll * cu_count) wpr *= 2;
  return wpr;
}

// Compute units of the current device, or `fallback` when no GPU is visible
// (the compile C-ABI also runs on build hosts).
int device_cu_count(int fallback) {
  int n = 0, dev = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || hipGetDevice(&dev) != hipSuccess) return fallback;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess || prop.multiProcessorCount <= 0) return fallback;
  return prop.multiProcessorCount;
}

// Dynamic LDS added to an exchange kernel (wave layout `ks`) so that no CU
// holds two of its workgroups (spreads a grid of <= CU-count tiles over all
// CUs).
int exchange_lds_pad(int in_dt, int out_dt, int loaders) {
  const int stat = chain_kernel_lds_bytes(in_dt, out_dt, loaders);
  const int want = 80 * 1024 + 1024;
  return stat >= want ? 0 : want - stat;
}

static_assert(kExchangeMaxTiles == kMaxExchangeTiles, "exchange slot limit");
}  // namespace wtc

namespace {

using namespace wtc;

constexpr int kTile = 128;            // BN of chain_tile_kernel, rows of the exchange tiles
constexpr int kRescaleRowsPerWg = 4;  // rescale_rows_kernel
constexpr int kMaxDevices = 64;
// Timeout mailbox words per device: slot 0 is shared by the streams that
// found every other slot taken, slots 1.. belong to one stream each.
constexpr int kMailboxSlots = 64;
constexpr int64_t kMinDefaultWorkspace = 1 << 20;

thread_local std::string g_last_error;
std::atomic<uint64_t> g_spin_ticks{0};  // 0: derived from the plan's estimate

// Limit of one exchange-path wait, in 100 MHz ticks: the caller's setting,
// else 200 times the cost model's estimate of the whole call, at least 5 ms
// (a wait of tiles that are all resident ends within the kernel's duration;
// the floor leaves room for launch skew and time-slicing with other
// processes) and at most 2 s.
uint64_t wait_limit_ticks(double est_us) {
  const uint64_t set = g_spin_ticks.load();
  if (set) return set;
  double us = 200.0 * est_us;
  if (!(us >= 5000.0)) us = 5000.0;
  if (us > 2.0e6) us = 2.0e6;
  return (uint64_t)(us * 100.0);
}

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

bool valid_in(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16 || dt == DT_FP8; }
bool valid_out(int dt) { return dt == DT_F32 || dt == DT_F16 || dt == DT_BF16; }

// Workspace layout (bytes).  The slot generation words sit at a fixed place
// with a fixed size, and a slot's exchange entries at a fixed place
// (slot * 1 KiB into the statistics region), so a workspace reused across
// problem shapes never mistakes another call's data for its own.
//   [0, 256)                 diagnostic words (flags, longest wait, timeouts)
//   [256, 256 + 4 KiB)       exchange slot generation words
//   [.., +stats)             split: float2 [batch][rows padded to 256][nT];
//                            exchange: uint64 [tiles][128] tagged entries
//   [.., +logits)            unfused path only: f32 logits, row max, row sum
constexpr int64_t kGenOff = 256;
constexpr int64_t kGenBytes = (int64_t)kMaxExchangeTiles * 4;

struct WsLayout {
  int64_t gen_off, stats_off, stats_bytes;
  int64_t logits_off, max_off, sum_off;
  int64_t total;
};

WsLayout ws_layout(int64_t batch, int64_t m, int64_t n, int path) {
  WsLayout w{};
  const int64_t nT = ceil_div(n, kTile);
  w.gen_off = kGenOff;
  w.stats_off = align256(kGenOff + kGenBytes);
  // split statistics rows padded to 256 per batch (either tile height)
  const int64_t split_bytes = batch * ceil_div(m, 256) * 256 * nT * 8;
  const int64_t exch_bytes = batch * ceil_div(m, kTile) * nT * kTile * 8;
  w.stats_bytes = align256(split_bytes > exch_bytes ? split_bytes : exch_bytes);
  w.total = w.stats_off + w.stats_bytes;
  if (path == WTC_PATH_UNFUSED) {
    w.logits_off = w.total;
    w.max_off = w.logits_off + align256(batch * m * n * 4);
    w.sum_off = w.max_off + align256(batch * m * 4);
    w.total = w.sum_off + align256(batch * m * 4);
  }
  return w;
}

int check_args(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dt, int out_dt,
               int path) {
  if (batch < 0 || m < 0 || n < 0 || k < 0)
    return fail(WTC_ERR_ARG, "negative extent");
  if (!valid_in(in_dt)) return fail(WTC_ERR_ARG, "unsupported in_dtype");
  if (!valid_out(out_dt)) return fail(WTC_ERR_ARG, "unsupported out_dtype");
  if (path < WTC_PATH_AUTO || path > WTC_PATH_ROWS)
    return fail(WTC_ERR_ARG, "unknown path");
  if ((k * dtype_bytes(in_dt)) % 16 != 0)
    return fail(WTC_ERR_ARG, "k * element bytes must be a multiple of 16");
  if (n % 8 != 0) return fail(WTC_ERR_ARG, "n must be a multiple of 8");
  // Buffer descriptors address one batch slice of A, B, out with 32-bit offsets.
  const int64_t isz = dtype_bytes(in_dt), osz = dtype_bytes(out_dt);
  const int64_t lim = 0x7FFFFFFFll;
  if (m * k * isz > lim || k * n * isz > lim || m * n * osz > lim || m * n * 4 > lim)
    return fail(WTC_ERR_UNSUPPORTED, "one batch slice of A, B or out exceeds 2 GiB");
  return WTC_OK;
}

struct Plan {
  VariantDesc v{};
  int path = 0;
  int64_t grid = 0, ws = 0;
  double est_us = 0;
};

std::string tiles_text(const wtc_tiles& t) {
  return std::to_string(t.tile_m) + "x" + std::to_string(t.tile_n) + "x" + std::to_string(t.tile_k) +
         "/" + std::to_string(t.thread_tile_m) + "x" + std::to_string(t.thread_tile_n);
}

// The variant and path to run: the cost model's first choice among the
// variants allowed (`tiles`, or all) and the paths allowed (`path`; AUTO =
// the fused ones).  `xch_per_cu`: exchange-kernel workgroups one CU holds.
int plan_impl(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dt, int out_dt, int path,
              const wtc_tiles* tiles, int cu_count, int xch_per_cu, Plan* out) {
  int rc = check_args(batch, m, n, k, in_dt, out_dt, path);
  if (rc) return rc;
  if (cu_count <= 0) return fail(WTC_ERR_ARG, "cu_count must be positive");
  int vid = -1;
  if (tiles) {
    VariantDesc v;
    if (!find_variant(in_dt, tiles->tile_m, tiles->tile_n, tiles->tile_k, tiles->thread_tile_m,
                      tiles->thread_tile_n, &v)) {
      std::string msg = "no gfx950 kernel variant has tiles " + tiles_text(*tiles) +
                        " for this input type; available:";
      for (const VariantDesc& d : variants_for(in_dt))
        msg += " " + tiles_text(wtc_tiles{d.tile_m, d.tile_n, d.tile_k, d.thread_tile_m, d.thread_tile_n});
      return fail(WTC_ERR_UNSUPPORTED, msg);
    }
    vid = v.id;
  }
  const Problem pr{batch, m, n, k, in_dt, out_dt, cu_count, xch_per_cu};
  Choice c{};
  if (!best_choice(pr, path, vid, &c)) {
    // the reason of the first variant that implements the path asked for
    std::string why = "no kernel variant runs this problem";
    for (const VariantDesc& d : variants_for(in_dt)) {
      if (vid >= 0 && d.id != vid) continue;
      const int q = path == WTC_PATH_AUTO ? WTC_PATH_SPLIT : path;
      const std::string r = infeasible_reason(d, q, pr);
      if (!r.empty()) {
        why = r;
        if (d.paths & (1u << q)) break;
      }
    }
    return fail(WTC_ERR_UNSUPPORTED, why);
  }
  const int64_t grid = variant_grid(c.v, c.path, pr);
  if (grid > 0x7FFFFFFFll) return fail(WTC_ERR_UNSUPPORTED, "too many tiles for one grid");
  out->v = c.v;
  out->path = c.path;
  out->grid = grid;
  out->ws = ws_layout(batch, m, n, c.path).total;
  out->est_us = c.est_us;
  return WTC_OK;
}

// Recent plans of the launch path, keyed by everything plan_impl reads:
// callers repeat shapes, and ranking the variants on every call costs a few
// microseconds of host time.  Guarded by g_mu.
struct PlanKey {
  int64_t batch, m, n, k;
  int in_dt, out_dt, path, cu, occ;
  int64_t tiles[5];  // all zero: no variant given
  bool operator==(const PlanKey& o) const { return std::memcmp(this, &o, sizeof *this) == 0; }
};
struct PlanCache {
  static constexpr int kSize = 16;
  PlanKey key[kSize];
  Plan plan[kSize];
  int used = 0, next = 0;
  const Plan* find(const PlanKey& k) const {
    for (int i = 0; i < used; ++i)
      if (key[i] == k) return &plan[i];
    return nullptr;
  }
  void put(const PlanKey& k, const Plan& p) {
    key[next] = k;
    plan[next] = p;
    next = (next + 1) % kSize;
    if (used < kSize) ++used;
  }
};
PlanCache g_plans;

PlanKey plan_key(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dt, int out_dt, int path,
                 const wtc_tiles* tiles, int cu, int occ) {
  PlanKey key;
  std::memset(&key, 0, sizeof key);  // padding too: keys compare bytewise
  key.batch = batch;
  key.m = m;
  key.n = n;
  key.k = k;
  key.in_dt = in_dt;
  key.out_dt = out_dt;
  key.path = path;
  key.cu = cu;
  key.occ = occ;
  if (tiles) {
    key.tiles[0] = tiles->tile_m;
    key.tiles[1] = tiles->tile_n;
    key.tiles[2] = tiles->tile_k;
    key.tiles[3] = tiles->thread_tile_m;
    key.tiles[4] = tiles->thread_tile_n;
  }
  return key;
}

// A default workspace of one stream.  Grow-only: a superseded buffer is kept
// (in `retired`) until the process ends, because a graph captured earlier may
// still hold its address.
struct StreamWorkspace {
  hipStream_t stream;
  void* ptr;
  size_t bytes;
};
struct RetiredBuffer {
  hipStream_t stream;
  void* ptr;
};

struct DeviceState {
  bool init = false;
  int cu_count = 0;
  int occ[4][3] = {};  // exchange-kernel workgroups per CU (fewest of the layouts), [in_dt][out_dt]
  std::vector<StreamWorkspace> ws;
  std::vector<RetiredBuffer> retired;
  // Host-visible words the exchange kernels set when a wait times out
  // (pinned, mapped host memory, kMailboxSlots words), one per stream: the
  // next call on the stream of the timed-out call reports it.
  volatile uint32_t* mailbox_host = nullptr;
  uint32_t* mailbox_dev = nullptr;
  hipStream_t slot_stream[kMailboxSlots] = {};
  bool slot_used[kMailboxSlots] = {};
  // Cross-stream ordering of exchange-path calls: an event recorded after
  // every exchange launch, and the stream it was recorded on.
  hipEvent_t exch_event = nullptr;
  hipStream_t exch_stream = nullptr;
  bool exch_used = false;
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];

#define HIP_TRY(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return fail(WTC_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)


// The device's state.  `host_objects`: also create the timeout mailbox
// (pinned host memory) and the exchange event, which the allocation-free
// entry point never does itself (it uses them when an earlier call made them).
int device_state(int dev, DeviceState** out, bool host_objects = true) {
  if (dev < 0 || dev >= kMaxDevices) return fail(WTC_ERR_HIP, "device index out of range");
  DeviceState& s = g_dev[dev];
  if (!s.init) {
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    s.cu_count = prop.multiProcessorCount;
    if (rows_kernel_max_k() != kRowsMaxK)
      return fail(WTC_ERR_HIP, "the rows kernel's k limit differs from the variant table's");
    for (int i = 0; i < 4; ++i)
      for (int o = 0; o < 3; ++o) {
        s.occ[i][o] = 1 << 30;
        for (int lw = 0; lw <= 1; ++lw) {
          const void* fn = chain_kernel_symbol(i, o, kEpiExchange, 128, lw);
          if (!fn) continue;  // f32 has no loader-wave layout
          const int pad = exchange_lds_pad(i, o, lw);
          HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, pad));
          int nb = 0;
          HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, chain_kernel_threads(i), pad));
          if (nb < s.occ[i][o]) s.occ[i][o] = nb;
        }
      }
    s.init = true;
  }
  if (host_objects && !s.mailbox_host) {
    void* mb = nullptr;
    HIP_TRY(hipHostMalloc(&mb, kMailboxSlots * sizeof(uint32_t),
                          hipHostMallocMapped | hipHostMallocCoherent));
    std::memset(mb, 0, kMailboxSlots * sizeof(uint32_t));
    void* mbd = nullptr;
    HIP_TRY(hipHostGetDevicePointer(&mbd, mb, 0));
    s.mailbox_host = static_cast<volatile uint32_t*>(mb);
    s.mailbox_dev = static_cast<uint32_t*>(mbd);
    // ordering between streams of one device only: no system-scope fence
    HIP_TRY(hipEventCreateWithFlags(&s.exch_event, hipEventDisableTiming | hipEventDisableSystemFence));
  }
  *out = &s;
  return WTC_OK;
}

int zero_fill(void* p, int64_t bytes, hipStream_t stream) {
  const int64_t words = bytes / 4;
  if (words <= 0) return WTC_OK;
  int64_t blocks = ceil_div(words, 256);
  if (blocks > 4096) blocks = 4096;
  uint32_t* ptr = static_cast<uint32_t*>(p);
  int64_t n = words;
  void* args[] = {&ptr, &n};
  HIP_TRY(hipLaunchKernel(zero_kernel_symbol(), dim3((unsigned)blocks), dim3(256), args, 0, stream));
  return WTC_OK;
}

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) != hipSuccess) return false;
  return st != hipStreamCaptureStatusNone;
}

// The default workspace of `stream` with at least `need` bytes, zeroed on
// that stream when first allocated.  No allocation while the stream is being
// captured into a graph.
int default_workspace(DeviceState* s, int64_t need, void** ws, hipStream_t stream) {
  StreamWorkspace* cur = nullptr;
  for (StreamWorkspace& w : s->ws)
    if (w.stream == stream) cur = &w;
  if (cur && (int64_t)cur->bytes >= need) {
    *ws = cur->ptr;
    return WTC_OK;
  }
  if (stream_capturing(stream))
    return fail(WTC_ERR_ARG,
                "the stream is being captured and its default workspace would have to be "
                "allocated: pass a workspace, or make one call of this shape on this stream "
                "before capturing");
  const int64_t bytes = need < kMinDefaultWorkspace ? kMinDefaultWorkspace : need;
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, (size_t)bytes));
  int rc = zero_fill(p, bytes, stream);
  if (rc) {
    (void)hipFree(p);
    return rc;
  }
  if (cur) {
    s->retired.push_back(RetiredBuffer{stream, cur->ptr});
    cur->ptr = p;
    cur->bytes = (size_t)bytes;
  } else {
    s->ws.push_back(StreamWorkspace{stream, p, (size_t)bytes});
  }
  *ws = p;
  return WTC_OK;
}

int launch_chain(const void* kern, int threads, int64_t grid, int lds_dyn,
                 const ChainParams& prm, hipStream_t stream) {
  ChainParams p = prm;
  void* args[] = {&p};
  HIP_TRY(hipLaunchKernel(kern, dim3((unsigned)grid), dim3(threads), args, (size_t)lds_dyn, stream));
  return WTC_OK;
}

// The tile kernel of a variant for an epilogue (NULL when not built), and
// its workgroup size.
struct TileKernel {
  const void* fn;
  int threads;
};
TileKernel tile_kernel(const VariantDesc& v, int in_dt, int out_dt, int epi) {
  if (v.id == kVarTile256x256) return {wide_kernel_symbol(in_dt, out_dt, epi), wide_kernel_threads()};
  return {chain_kernel_symbol(in_dt, out_dt, epi, v.tile_rows, v.loaders), chain_kernel_threads(in_dt)};
}

// chain_tile_kernel: the scalars a tile needs before its first load lead the
// argument list (preloaded into SGPRs), then the parameter block.  check_args
// keeps every batch slice below 2 GiB, so the 32-bit sizes and strides hold.
// `done`, if given, is an event that completes with the kernel: attached to
// the launch itself (hipExtLaunchKernel), it costs nothing, where a separate
// hipEventRecord after the launch adds a gap of 1-3 us between kernels.
int launch_tile(const void* kern, int threads, int64_t grid, int lds_dyn,
                const ChainParams& prm, hipStream_t stream, hipEvent_t done = nullptr) {
  if (!kern) return fail(WTC_ERR_UNSUPPORTED, "no kernel built for this variant and path");
  ChainParams p = prm;
  const uint8_t* a = p.a;
  const uint8_t* b = p.b;
  uint32_t M = (uint32_t)p.M, N = (uint32_t)p.N, K = (uint32_t)p.K;
  uint32_t lda = (uint32_t)p.lda_bytes, ldb = (uint32_t)p.ldb_bytes;
  uint32_t nT = (uint32_t)p.nT, nRB = (uint32_t)p.nRB;
  uint32_t a_bs = (uint32_t)p.a_bstride, b_bs = (uint32_t)p.b_bstride;
  uint32_t g = (uint32_t)grid;
  void* args[] = {&a, &b, &M, &N, &K, &lda, &ldb, &nT, &nRB, &a_bs, &b_bs, &g, &p};
  if (done)
    HIP_TRY(hipExtLaunchKernel(kern, dim3((unsigned)grid), dim3(threads), args, (size_t)lds_dyn,
                               stream, nullptr, done, 0));
  else
    HIP_TRY(hipLaunchKernel(kern, dim3((unsigned)grid), dim3(threads), args, (size_t)lds_dyn, stream));
  return WTC_OK;
}

// The mailbox slot of `stream`: its own, given out on its first call, or
// slot 0, shared by the streams that came when all others were taken.  The
// table is a fixed array: looking a stream up allocates nothing.
int mailbox_slot(DeviceState* ds, hipStream_t stream) {
  for (int i = 1; i < kMailboxSlots; ++i)
    if (ds->slot_used[i] && ds->slot_stream[i] == stream) return i;
  for (int i = 1; i < kMailboxSlots; ++i)
    if (!ds->slot_used[i]) {
      ds->slot_used[i] = true;
      ds->slot_stream[i] = stream;
      if (ds->mailbox_host) ds->mailbox_host[i] = 0u;
      return i;
    }
  return 0;
}

// The device address of `stream`'s mailbox word (NULL while the device has
// no mailbox: the allocation-free entry point does not create it).
uint32_t* mailbox_word(DeviceState* ds, hipStream_t stream) {
  if (!ds->mailbox_dev) return nullptr;
  return ds->mailbox_dev + mailbox_slot(ds, stream);
}

// A timed-out exchange wait of an earlier call on `stream`, reported once.
// Seen once that call's kernel has finished, so the first call on the stream
// made after that (or wtc_check_status, which synchronises the stream first)
// reports it.
int take_mailbox(DeviceState* ds, hipStream_t stream) {  // no mailbox yet: nothing to report
  if (!ds->mailbox_host) return WTC_OK;
  uint32_t* word = const_cast<uint32_t*>(ds->mailbox_host) + mailbox_slot(ds, stream);
  if (*word != 0u && __atomic_exchange_n(word, 0u, __ATOMIC_SEQ_CST) != 0u) {
    return fail(WTC_ERR_TIMEOUT,
                "an exchange-path wait of an earlier call on this stream timed out (its tiles "
                "were not all resident at once); that call's output is wrong");
  }
  return WTC_OK;
}

// Gives `stream`'s mailbox slot back (a timeout still in it is dropped).
void release_slot(DeviceState* ds, hipStream_t stream) {
  for (int i = 1; i < kMailboxSlots; ++i)
    if (ds->slot_used[i] && ds->slot_stream[i] == stream) {
      ds->slot_used[i] = false;
      ds->slot_stream[i] = nullptr;
      if (ds->mailbox_host) ds->mailbox_host[i] = 0u;
    }
}

// Frees what the library holds for `stream` (its default workspace and the
// buffers that one superseded) and gives its mailbox slot back.  The caller
// has synchronised the stream; graphs captured on it that use its default
// workspace must not be replayed afterwards.
int release_stream_state(DeviceState* ds, hipStream_t stream) {
  release_slot(ds, stream);
  if (ds->exch_stream == stream) ds->exch_stream = nullptr;
  for (size_t i = 0; i < ds->ws.size();) {
    if (ds->ws[i].stream == stream) {
      HIP_TRY(hipFree(ds->ws[i].ptr));
      ds->ws.erase(ds->ws.begin() + (long)i);
    } else {
      ++i;
    }
  }
  for (size_t i = 0; i < ds->retired.size();) {
    if (ds->retired[i].stream == stream) {
      HIP_TRY(hipFree(ds->retired[i].ptr));
      ds->retired.erase(ds->retired.begin() + (long)i);
    } else {
      ++i;
    }
  }
  return WTC_OK;
}

// Exchange-path calls on one device must not overlap (each needs all of its
// tiles resident).  Calls from this process on different streams are put in
// order: every exchange launch completes the device's exchange event, and a
// call on another stream first waits for it.  Not done for streams being
// captured into a graph (an event completed outside a capture cannot order
// it, nor can the capture complete it).
int launch_exchange(DeviceState* ds, const void* kern, int threads, int64_t grid, int lds_dyn,
                    const ChainParams& p, hipStream_t stream) {
  if (!ds->exch_event || stream_capturing(stream))
    return launch_tile(kern, threads, grid, lds_dyn, p, stream);
  if (ds->exch_used && stream != ds->exch_stream)
    HIP_TRY(hipStreamWaitEvent(stream, ds->exch_event, 0));
  const int rc = launch_tile(kern, threads, grid, lds_dyn, p, stream, ds->exch_event);
  if (rc) return rc;
  ds->exch_used = true;
  ds->exch_stream = stream;
  return WTC_OK;
}

// ---- scratch of the allocation-free entry point ------------------------------
// A file-scope device array, zeroed when the code object is loaded on a GPU
// (every GPU holds its own copy until the process ends).  Host code never
// passes `scratch` itself to a kernel or a copy: its address on a device is
// taken once with hipGetSymbolAddress (with that device current) and kept per
// device.  Nothing in it needs clearing between calls: the exchange path's
// slot generation words start at zero with the array and stay consistent
// across calls of any shape, and every other region is written before it is
// read within a call.
static __device__ __align__(256) uint8_t scratch[WTC_NOALLOC_SCRATCH_BYTES];
void* g_scratch[kMaxDevices] = {};

int scratch_address(int dev, void** out) {
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(WTC_ERR_HIP, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return WTC_OK;
}

int matmul_softmax_impl(const void* a, const void* b, void* out, int64_t batch, int64_t m,
                        int64_t n, int64_t k, int in_dtype, int out_dtype, float logit_scale,
                        float scale_a, float scale_b, const wtc_tiles* tiles, int path,
                        void* workspace, size_t workspace_bytes, void* stream_, bool noalloc);

// Profiling inputs: element i of a buffer of `dtype` from a hash of (seed, i),
// finite and within +-2 (f32, f16, bf16: sign, an exponent of 2^-7 .. 2^0 and
// random mantissa bits; fp8 e4m3: exponent field 1 .. 8, never the NaN code).
__global__ void fill_random_kernel(uint8_t* p, int64_t count, int dtype, uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    uint64_t h = seed ^ ((uint64_t)i * 0x9E3779B97F4A7C15ull);
    h ^= h >> 31;
    h *= 0xBF58476D1CE4E5B9ull;
    h ^= h >> 29;
    const uint32_t r = (uint32_t)(h >> 16);
    const uint32_t sign = r >> 31, mant = r & 0x7FFFFFu, ex = (r >> 23) & 7u;
    if (dtype == DT_FP8) {
      p[i] = (uint8_t)((sign << 7) | ((ex + 1u) << 3) | (mant & 7u));
      continue;
    }
    const uint32_t bits = (sign << 31) | ((127u - 7u + ex) << 23) | mant;
    if (dtype == DT_F32) {
      reinterpret_cast<uint32_t*>(p)[i] = bits;
    } else if (dtype == DT_BF16) {
      reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)(bits >> 16);
    } else {  // f16: exponent 15 - 7 + ex, top ten mantissa bits
      reinterpret_cast<uint16_t*>(p)[i] =
          (uint16_t)((sign << 15) | ((15u - 7u + ex) << 10) | (mant >> 13));
    }
  }
}

}  // namespace

extern "C" {

const char* wtc_last_error(void) { return g_last_error.c_str(); }

const char* wtc_version(void) { return "wtc-mi355x 0.2.0 (gfx950)"; }

int wtc_plan(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype, int out_dtype,
             int path, int cu_count, int wg_per_cu, int64_t* grid, int* chosen_path,
             int64_t* workspace_bytes) {
  return wtc_plan_tiles(batch, m, n, k, in_dtype, out_dtype, path, nullptr, cu_count, wg_per_cu,
                        nullptr, chosen_path, grid, workspace_bytes, nullptr);
}

int wtc_plan_tiles(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype, int out_dtype,
                   int path, const wtc_tiles* tiles, int cu_count, int wg_per_cu,
                   wtc_tiles* chosen_tiles, int* chosen_path, int64_t* grid,
                   int64_t* workspace_bytes, double* estimated_us) {
  g_last_error.clear();
  Plan pl;
  const int rc = plan_impl(batch, m, n, k, in_dtype, out_dtype, path, tiles, cu_count, wg_per_cu, &pl);
  if (rc) return rc;
  if (chosen_tiles)
    *chosen_tiles = wtc_tiles{pl.v.tile_m, pl.v.tile_n, pl.v.tile_k, pl.v.thread_tile_m, pl.v.thread_tile_n};
  if (chosen_path) *chosen_path = pl.path;
  if (grid) *grid = pl.grid;
  if (workspace_bytes) *workspace_bytes = pl.ws;
  if (estimated_us) *estimated_us = pl.est_us;
  return WTC_OK;
}

int wtc_profile_tiles(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype, int out_dtype,
                      const wtc_tiles* tiles, int path, int warmup, int iters, uint64_t seed,
                      double* us_per_call) {
  g_last_error.clear();
  if (!us_per_call) return fail(WTC_ERR_ARG, "us_per_call is NULL");
  if (iters <= 0 || warmup < 0) return fail(WTC_ERR_ARG, "iters must be positive, warmup >= 0");
  int rc = check_args(batch, m, n, k, in_dtype, out_dtype, path);
  if (rc) return rc;
  if (batch == 0 || m == 0 || n == 0) return fail(WTC_ERR_ARG, "empty problem");
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  int cu = 0, occ = 1;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState* ds = nullptr;
    rc = device_state(dev, &ds);
    if (rc) return rc;
    cu = ds->cu_count;
    occ = ds->occ[in_dtype][out_dtype];
  }
  Plan pl;
  rc = plan_impl(batch, m, n, k, in_dtype, out_dtype, path, tiles, cu, occ, &pl);
  if (rc) return rc;
  const int64_t isz = dtype_bytes(in_dtype), osz = dtype_bytes(out_dtype);
  const size_t a_bytes = (size_t)(batch * m * k * isz), b_bytes = (size_t)(batch * k * n * isz);
  const size_t o_bytes = (size_t)(batch * m * n * osz), w_bytes = (size_t)pl.ws;
  void *a = nullptr, *b = nullptr, *o = nullptr, *w = nullptr;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  auto release = [&]() {
    if (st) {
      (void)hipStreamSynchronize(st);
      std::lock_guard<std::mutex> lk(g_mu);
      (void)release_stream_state(&g_dev[dev], st);
    }
    for (void* q : {a, b, o, w})
      if (q) (void)hipFree(q);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
  };
  auto run = [&]() -> int {
    HIP_TRY(hipMalloc(&a, a_bytes ? a_bytes : 16));
    HIP_TRY(hipMalloc(&b, b_bytes ? b_bytes : 16));
    HIP_TRY(hipMalloc(&o, o_bytes));
    HIP_TRY(hipMalloc(&w, w_bytes));
    HIP_TRY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    int r = zero_fill(w, (int64_t)w_bytes, st);
    if (r) return r;
    const struct { void* p; int64_t count; uint64_t salt; } fills[] = {
        {a, batch * m * k, 0x5851F42D4C957F2Dull}, {b, batch * k * n, 0x14057B7EF767814Full}};
    for (const auto& f : fills) {
      if (f.count == 0) continue;
      uint8_t* ptr = static_cast<uint8_t*>(f.p);
      int64_t count = f.count;
      int dt = in_dtype;
      uint64_t sd = seed ^ f.salt;
      void* args[] = {&ptr, &count, &dt, &sd};
      HIP_TRY(hipLaunchKernel(reinterpret_cast<const void*>(&fill_random_kernel), dim3(1024),
                              dim3(256), args, 0, st));
    }
    for (int i = 0; i < warmup + iters; ++i) {
      if (i == warmup) HIP_TRY(hipEventRecord(e0, st));
      r = matmul_softmax_impl(a, b, o, batch, m, n, k, in_dtype, out_dtype, 1.0f, 1.0f, 1.0f,
                              tiles, path, w, w_bytes, st, false);
      if (r) return r;
    }
    HIP_TRY(hipEventRecord(e1, st));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    *us_per_call = (double)ms * 1e3 / iters;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState* ds = nullptr;
    r = device_state(dev, &ds);
    return r ? r : take_mailbox(ds, st);
  };
  rc = run();
  const std::string msg = g_last_error;
  release();
  g_last_error = msg;
  return rc;
}

int wtc_list_variants(int in_dtype, wtc_tiles* tiles, unsigned* paths, const char** names,
                      int capacity) {
  g_last_error.clear();
  if (!valid_in(in_dtype)) {
    fail(WTC_ERR_ARG, "unsupported in_dtype");
    return -1;
  }
  const std::vector<VariantDesc> vs = variants_for(in_dtype);
  for (int i = 0; i < (int)vs.size() && i < capacity; ++i) {
    const VariantDesc& v = vs[i];
    if (tiles) tiles[i] = wtc_tiles{v.tile_m, v.tile_n, v.tile_k, v.thread_tile_m, v.thread_tile_n};
    if (paths) paths[i] = v.paths;
    if (names) names[i] = v.name;
  }
  return (int)vs.size();
}

int64_t wtc_matmul_softmax_workspace_size(int64_t batch, int64_t m, int64_t n, int64_t k,
                                          int in_dtype, int out_dtype, int path) {
  g_last_error.clear();
  if (check_args(batch, m, n, k, in_dtype, out_dtype, path)) return -1;
  return ws_layout(batch, m, n, path).total;
}

int wtc_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (!workspace && workspace_bytes) return fail(WTC_ERR_ARG, "workspace is NULL");
  return zero_fill(workspace, (int64_t)workspace_bytes, static_cast<hipStream_t>(stream));
}

int wtc_set_exchange_wait_limit(uint64_t ticks) {
  g_last_error.clear();
  g_spin_ticks.store(ticks);
  return WTC_OK;
}

int wtc_check_status(void* stream_) {
  g_last_error.clear();
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  HIP_TRY(hipStreamSynchronize(stream));
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* ds = nullptr;
  int rc = device_state(dev, &ds);
  if (rc) return rc;
  // the allocation-free entry point's set-up too, so that its calls after
  // this one do none (they may then be captured into a graph)
  void* scratch_ptr = nullptr;
  rc = scratch_address(dev, &scratch_ptr);
  if (rc) return rc;
  return take_mailbox(ds, stream);
}

int wtc_release_stream(void* stream_) {
  g_last_error.clear();
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(WTC_ERR_HIP, "device index out of range");
  HIP_TRY(hipStreamSynchronize(stream));
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* ds = &g_dev[dev];
  const int rc = ds->mailbox_host ? take_mailbox(ds, stream) : WTC_OK;
  const std::string msg = g_last_error;
  const int frc = release_stream_state(ds, stream);
  if (frc) return frc;
  g_last_error = msg;
  return rc;
}

int wtc_read_error_flags(void* workspace, uint32_t* flags, int clear) {
  g_last_error.clear();
  if (!flags) return fail(WTC_ERR_ARG, "flags is NULL");
  flags[0] = flags[1] = flags[2] = 0;
  std::vector<void*> bufs;
  if (workspace) {
    bufs.push_back(workspace);
  } else {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(WTC_ERR_HIP, "device index out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    for (const StreamWorkspace& w : g_dev[dev].ws) bufs.push_back(w.ptr);
    if (g_scratch[dev]) bufs.push_back(g_scratch[dev]);
  }
  HIP_TRY(hipDeviceSynchronize());
  for (void* b : bufs) {
    uint32_t w[3];
    HIP_TRY(hipMemcpy(w, b, sizeof w, hipMemcpyDeviceToHost));
    flags[0] |= w[0];
    flags[1] = w[1] > flags[1] ? w[1] : flags[1];
    flags[2] += w[2];
    if (clear) {
      const uint32_t zero[3] = {0, 0, 0};
      HIP_TRY(hipMemcpy(b, zero, sizeof zero, hipMemcpyHostToDevice));
    }
  }
  return WTC_OK;
}

int wtc_matmul_softmax(const void* a, const void* b, void* out, int64_t batch, int64_t m,
                       int64_t n, int64_t k, int in_dtype, int out_dtype, float logit_scale,
                       float scale_a, float scale_b, int path, void* workspace,
                       size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  return matmul_softmax_impl(a, b, out, batch, m, n, k, in_dtype, out_dtype, logit_scale, scale_a,
                             scale_b, nullptr, path, workspace, workspace_bytes, stream, false);
}

int wtc_matmul_softmax_tiles(const void* a, const void* b, void* out, int64_t batch, int64_t m,
                             int64_t n, int64_t k, int in_dtype, int out_dtype, float logit_scale,
                             float scale_a, float scale_b, const wtc_tiles* tiles, int path,
                             void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  return matmul_softmax_impl(a, b, out, batch, m, n, k, in_dtype, out_dtype, logit_scale, scale_a,
                             scale_b, tiles, path, workspace, workspace_bytes, stream, false);
}

int wtc_matmul_softmax_noalloc(const void* a, const void* b, void* out, int64_t batch, int64_t m,
                               int64_t n, int64_t k, int in_dtype, int out_dtype,
                               float logit_scale, float scale_a, float scale_b, int path,
                               void* stream) {
  g_last_error.clear();
  return matmul_softmax_impl(a, b, out, batch, m, n, k, in_dtype, out_dtype, logit_scale, scale_a,
                             scale_b, nullptr, path, nullptr, 0, stream, true);
}

}  // extern "C"

namespace {

int matmul_softmax_impl(const void* a, const void* b, void* out, int64_t batch, int64_t m,
                        int64_t n, int64_t k, int in_dtype, int out_dtype, float logit_scale,
                        float scale_a, float scale_b, const wtc_tiles* tiles, int path,
                        void* workspace, size_t workspace_bytes, void* stream_, bool noalloc) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc = check_args(batch, m, n, k, in_dtype, out_dtype, path);
  if (rc) return rc;
  if (batch == 0 || m == 0 || n == 0) return WTC_OK;
  if (!out || (k > 0 && (!a || !b))) return fail(WTC_ERR_ARG, "null data pointer");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(out)) & 15u)
    return fail(WTC_ERR_ARG, "data pointers must be 16-byte aligned");
  if (!std::isfinite(logit_scale) || !std::isfinite(scale_a) || !std::isfinite(scale_b))
    return fail(WTC_ERR_ARG, "scales must be finite");

  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  // The lock covers the shared state (device state, plan cache, default
  // workspaces, mailbox, the exchange path's cross-stream event); the
  // launches of the other paths only read this call's own values, so they
  // run unlocked and calls from several host threads enqueue in parallel.
  std::unique_lock<std::mutex> lk(g_mu);
  DeviceState* ds = nullptr;
  rc = device_state(dev, &ds, !noalloc);
  if (rc) return rc;
  rc = take_mailbox(ds, stream);
  if (rc) return rc;

  Plan pl;
  const PlanKey key = plan_key(batch, m, n, k, in_dtype, out_dtype, path, tiles, ds->cu_count,
                               ds->occ[in_dtype][out_dtype]);
  if (const Plan* hit = g_plans.find(key)) {
    pl = *hit;
  } else {
    rc = plan_impl(batch, m, n, k, in_dtype, out_dtype, path, tiles, ds->cu_count,
                   ds->occ[in_dtype][out_dtype], &pl);
    if (rc) return rc;
    g_plans.put(key, pl);
  }
  const int64_t grid = pl.grid, need = pl.ws;
  const int chosen = pl.path;
  const VariantDesc& var = pl.v;

  void* ws = workspace;
  if (noalloc) {
    if (need > (int64_t)WTC_NOALLOC_SCRATCH_BYTES)
      return fail(WTC_ERR_WORKSPACE,
                  "this problem needs " + std::to_string(need) +
                      " bytes of workspace; the allocation-free entry point has " +
                      std::to_string((int64_t)WTC_NOALLOC_SCRATCH_BYTES) +
                      " (use wtc_matmul_softmax with a workspace)");
    rc = scratch_address(dev, &ws);
    if (rc) return rc;
  } else if (ws) {
    if ((int64_t)workspace_bytes < need)
      return fail(WTC_ERR_WORKSPACE, "workspace needs " + std::to_string(need) + " bytes");
    if (reinterpret_cast<uintptr_t>(ws) & 255u)
      return fail(WTC_ERR_ARG, "workspace must be 256-byte aligned");
  } else {
    rc = default_workspace(ds, need, &ws, stream);
    if (rc) return rc;
  }
  const WsLayout L = ws_layout(batch, m, n, chosen);
  uint8_t* wsb = static_cast<uint8_t*>(ws);

  const int isz = dtype_bytes(in_dtype), osz = dtype_bytes(out_dtype);
  const float lin = logit_scale * scale_a * scale_b;
  ChainParams p{};
  p.a = static_cast<const uint8_t*>(a);
  p.b = static_cast<const uint8_t*>(b);
  p.out = static_cast<uint8_t*>(out);
  p.M = m;
  p.N = n;
  p.K = k;
  p.a_bstride = m * k * isz;
  p.b_bstride = k * n * isz;
  p.o_bstride = m * n * osz;
  p.lda_bytes = k * isz;
  p.ldb_bytes = n * isz;
  p.ldo_bytes = n * osz;
  p.c2 = lin * 1.4426950408889634f;
  p.lin_scale = lin;
  // row blocks per batch of the kernel that runs
  const int tile_rows = var.tile_rows;
  p.nRB = (int)ceil_div(m, tile_rows);
  // column tiles per row block: the variant's on the split and unfused paths
  p.nT = (int)ceil_div(n, chosen == WTC_PATH_SPLIT || chosen == WTC_PATH_UNFUSED ? var.tile_n : kTile);
  p.partial = reinterpret_cast<float2*>(wsb + L.stats_off);
  p.ent = reinterpret_cast<uint64_t*>(wsb + L.stats_off);
  p.gen = reinterpret_cast<uint32_t*>(wsb + L.gen_off);
  p.err = reinterpret_cast<uint32_t*>(wsb);
  p.mailbox = mailbox_word(ds, stream);
  p.spin_ticks = wait_limit_ticks(pl.est_us);

  const int cu_count = ds->cu_count;
  if (chosen != WTC_PATH_EXCHANGE) lk.unlock();
  if (chosen == WTC_PATH_ROWS) {
    return launch_chain(rows_kernel_symbol(in_dtype, out_dtype), rows_kernel_threads(), grid, 0,
                        p, stream);
  }
  if (chosen == WTC_PATH_EXCHANGE)
    return launch_exchange(ds, chain_kernel_symbol(in_dtype, out_dtype, kEpiExchange, 128, var.loaders),
                           chain_kernel_threads(in_dtype), grid,
                           exchange_lds_pad(in_dtype, out_dtype, var.loaders), p, stream);
  if (chosen == WTC_PATH_SPLIT) {
    const TileKernel tk = tile_kernel(var, in_dtype, out_dtype, kEpiSplit);
    rc = launch_tile(tk.fn, tk.threads, grid, 0, p, stream);
    if (rc) return rc;
    uint8_t* o = p.out;
    const float2* part = p.partial;
    // statistics rows per batch: the tile kernel's row blocks times its height
    int64_t rows_total = batch * m, M_ = m, rows_pad = (int64_t)p.nRB * tile_rows, N_ = n,
            ldo = p.ldo_bytes, ob = p.o_bstride;
    int nT = p.nT;
    int tshift = var.tile_n == 256 ? 8 : 7;  // log2 of the tile width
    int wpr = rescale_waves_per_row(rows_total, cu_count);
    void* args[] = {&o, &part, &rows_total, &M_, &rows_pad, &N_, &ldo, &ob, &nT, &tshift, &wpr};
    HIP_TRY(hipLaunchKernel(rescale_kernel_symbol(out_dtype),
                            dim3((unsigned)ceil_div(rows_total * wpr, kRescaleRowsPerWg)), dim3(256),
                            args, 0, stream));
    return WTC_OK;
  }
  // Unfused: logits (f32) into the workspace, then four row kernels.
  float* logits = reinterpret_cast<float*>(wsb + L.logits_off);
  float* rmax = reinterpret_cast<float*>(wsb + L.max_off);
  float* rsum = reinterpret_cast<float*>(wsb + L.sum_off);
  ChainParams q = p;
  q.out = reinterpret_cast<uint8_t*>(logits);
  q.o_bstride = m * n * 4;
  q.ldo_bytes = n * 4;
  const TileKernel tk = tile_kernel(var, in_dtype, DT_F32, kEpiLogits);
  rc = launch_tile(tk.fn, tk.threads, grid, 0, q, stream);
  if (rc) return rc;
  const int64_t rows = batch * m;
  if (rows > 0x7FFFFFFFll) return fail(WTC_ERR_UNSUPPORTED, "too many rows");
  int64_t N_ = n;
  {
    void* args[] = {&logits, &rmax, &N_};
    HIP_TRY(hipLaunchKernel(rowmax_kernel_symbol(), dim3((unsigned)rows), dim3(256), args, 0, stream));
  }
  {
    void* args[] = {&logits, &rmax, &N_};
    HIP_TRY(hipLaunchKernel(expsub_kernel_symbol(), dim3((unsigned)rows), dim3(256), args, 0, stream));
  }
  {
    void* args[] = {&logits, &rsum, &N_};
    HIP_TRY(hipLaunchKernel(rowsum_kernel_symbol(), dim3((unsigned)rows), dim3(256), args, 0, stream));
  }
  {
    void* o = out;
    void* args[] = {&logits, &rsum, &o, &N_};
    HIP_TRY(hipLaunchKernel(rowdiv_kernel_symbol(out_dtype), dim3((unsigned)rows), dim3(256), args, 0, stream));
  }
  return WTC_OK;
}

}  // namespace
