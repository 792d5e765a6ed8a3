// Block mask -> active-tile index lists, and the plan that owns them.
//
// The mask rule is evaluated on the GPU at token level and OR-reduced onto the
// 128x128 tile grid (one workgroup per tile pair), the bitmap is compacted to
// CSR by three small kernels (row popcount, single-workgroup scan, ordered
// fill), and the host derives the attention kernel's XCD-aware schedule (the
// units of each persistent workgroup) from the row lengths.
// Everything here runs once per shape; none of it is on the per-layer path.
#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <numeric>
#include <vector>

#include "common.h"
#include "plan.h"

namespace h3hip {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return H3HIP_EHIP;
  }
  return H3HIP_OK;
}

// ------------------------------------------------------------ rule on device

struct RuleDev {
  int32_t kind, seq_len, prefix_len, frames, height, width;
  int32_t frame_window, sp_h, sp_w, sp_window, band;
  int32_t n_tiles;
  const uint8_t* col_global;  // [n_tiles] BAND global columns
  const uint8_t* frame_landmark;  // [frames] landmark flags
};

__device__ __forceinline__ bool rule_allows(const RuleDev& r, int32_t q, int32_t k) {
  if (q >= r.seq_len || k >= r.seq_len) return false;
  if (r.kind == H3HIP_RULE_DENSE) return true;
  if (q < r.prefix_len || k < r.prefix_len) return true;
  const int32_t per = r.height * r.width;
  const int32_t vq = q - r.prefix_len, vk = k - r.prefix_len;
  const int32_t fq = vq / per, fk = vk / per;
  const int32_t pq = vq - fq * per, pk = vk - fk * per;
  const int32_t yq = pq / r.width, xq = pq - yq * r.width;
  const int32_t yk = pk / r.width, xk = pk - yk * r.width;
  if (r.kind == H3HIP_RULE_LOCAL) {
    if (abs(fq - fk) <= r.frame_window && abs(yq / r.sp_h - yk / r.sp_h) <= r.sp_window &&
        abs(xq / r.sp_w - xk / r.sp_w) <= r.sp_window)
      return true;
  } else {  // AXIAL
    if (fq == fk) return true;
    if (yq == yk && xq == xk) return true;
  }
  return r.frame_landmark != nullptr && r.frame_landmark[fk] != 0;
}

// One workgroup per tile pair; each thread tests a strided subset of the
// tile's token pairs and the workgroup ORs the answers.
__global__ __launch_bounds__(256) void mask_rule_kernel(RuleDev r, uint8_t* bitmap) {
  const int32_t qi = blockIdx.y, kj = blockIdx.x;
  uint8_t* dst = bitmap + (size_t)qi * r.n_tiles + kj;
  if (r.kind == H3HIP_RULE_BAND) {
    if (threadIdx.x == 0) *dst = (abs(qi - kj) <= r.band || r.col_global[kj]) ? 1 : 0;
    return;
  }
  const int32_t q0 = qi * H3HIP_TILE, k0 = kj * H3HIP_TILE;
  int hit = 0;
  for (int32_t pair = threadIdx.x; pair < H3HIP_TILE * H3HIP_TILE && !hit; pair += 256) {
    const int32_t q = q0 + (pair >> 7), k = k0 + (pair & 127);
    hit = rule_allows(r, q, k) ? 1 : 0;
  }
  hit = __syncthreads_or(hit);
  if (threadIdx.x == 0) *dst = hit ? 1 : 0;
}

// ------------------------------------------------------------- CSR kernels

// row_ptr[row + 1] = popcount(bitmap row); row_ptr[0] = 0.
__global__ __launch_bounds__(256) void row_count_kernel(const uint8_t* bitmap, int32_t nk,
                                                        int32_t* row_ptr) {
  const int32_t row = blockIdx.x;
  const uint8_t* src = bitmap + (size_t)row * nk;
  int cnt = 0;
  for (int32_t c = threadIdx.x; c < nk; c += 256) cnt += src[c] != 0;
  __shared__ int part[4];
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    row_ptr[row + 1] = part[0] + part[1] + part[2] + part[3];
    if (row == 0) row_ptr[0] = 0;
  }
}

// In-place inclusive scan of row_ptr[1..n] by one workgroup, 256 entries per pass.
__global__ __launch_bounds__(256) void scan_kernel(int32_t* row_ptr, int32_t n) {
  __shared__ int32_t buf[256];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int32_t base = 0; base < n; base += 256) {
    const int32_t i = base + threadIdx.x;
    int32_t v = i < n ? row_ptr[1 + i] : 0;
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      int32_t add = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
      __syncthreads();
      buf[threadIdx.x] += add;
      __syncthreads();
    }
    if (i < n) row_ptr[1 + i] = buf[threadIdx.x] + carry;
    __syncthreads();
    if (threadIdx.x == 255) carry += buf[255];
    __syncthreads();
  }
}

// Ordered compaction of one bitmap row into col_idx[row_ptr[row] ...].
__global__ __launch_bounds__(256) void fill_kernel(const uint8_t* bitmap, int32_t nk,
                                                   const int32_t* row_ptr, int32_t* col_idx) {
  const int32_t row = blockIdx.x;
  const uint8_t* src = bitmap + (size_t)row * nk;
  __shared__ int32_t wave_cnt[4];
  int32_t base = row_ptr[row];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int32_t c0 = 0; c0 < nk; c0 += 256) {
    const int32_t c = c0 + threadIdx.x;
    const bool on = c < nk && src[c] != 0;
    const uint64_t bal = __ballot(on);
    const int32_t before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = __popcll(bal);
    __syncthreads();
    int32_t off = 0;
    for (int w = 0; w < wave; w++) off += wave_cnt[w];
    if (on) col_idx[base + off + before] = c;
    const int32_t total = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
    base += total;
  }
}

// ------------------------------------------------------------ host helpers

static int validate_rule(const h3hip_mask_rule* r) {
  H3_REQUIRE(r != nullptr, H3HIP_EINVAL, "rule is NULL");
  H3_REQUIRE(r->seq_len > 0, H3HIP_EINVAL, "seq_len must be positive (got %d)", r->seq_len);
  H3_REQUIRE(r->kind >= H3HIP_RULE_DENSE && r->kind <= H3HIP_RULE_BITMAP, H3HIP_EINVAL,
             "unknown rule kind %d", r->kind);
  const int64_t n_tiles = (r->seq_len + H3HIP_TILE - 1) / H3HIP_TILE;
  H3_REQUIRE(n_tiles <= 32767, H3HIP_EINVAL, "seq_len %d exceeds the tile-index range",
             r->seq_len);
  if (r->kind == H3HIP_RULE_LOCAL || r->kind == H3HIP_RULE_AXIAL) {
    // AxialTopology refuses a lattice that does not fill the video span
    // (AxialTopology.swift:65-77) rather than index it wrongly.
    H3_REQUIRE(r->prefix_len >= 0 && r->frames > 0 && r->height > 0 && r->width > 0,
               H3HIP_EINVAL, "video lattice must be positive");
    H3_REQUIRE((int64_t)r->frames * r->height * r->width == (int64_t)r->seq_len - r->prefix_len,
               H3HIP_EINVAL, "lattice %dx%dx%d does not fill the video span [%d, %d)", r->frames,
               r->height, r->width, r->prefix_len, r->seq_len);
    H3_REQUIRE(r->n_landmarks >= 0 && (r->n_landmarks == 0 || r->landmark_frames != nullptr),
               H3HIP_EINVAL, "landmark_frames is NULL");
    for (int32_t i = 0; i < r->n_landmarks; i++)
      H3_REQUIRE(r->landmark_frames[i] >= 0 && r->landmark_frames[i] < r->frames, H3HIP_EINVAL,
                 "landmark frame %d outside [0, %d)", r->landmark_frames[i], r->frames);
  }
  if (r->kind == H3HIP_RULE_LOCAL)
    H3_REQUIRE(r->frame_window >= 0 && r->spatial_tile_h > 0 && r->spatial_tile_w > 0 &&
                   r->spatial_window >= 0,
               H3HIP_EINVAL, "local-window parameters must be non-negative with positive tiles");
  if (r->kind == H3HIP_RULE_BAND) {
    H3_REQUIRE(r->band >= 0, H3HIP_EINVAL, "band must be non-negative");
    H3_REQUIRE(r->n_global_cols >= 0 && (r->n_global_cols == 0 || r->global_cols != nullptr),
               H3HIP_EINVAL, "global_cols is NULL");
    for (int32_t i = 0; i < r->n_global_cols; i++)
      H3_REQUIRE(r->global_cols[i] >= 0 && r->global_cols[i] < n_tiles, H3HIP_EINVAL,
                 "global column %d outside [0, %lld)", r->global_cols[i], (long long)n_tiles);
  }
  if (r->kind == H3HIP_RULE_BITMAP)
    H3_REQUIRE(r->bitmap != nullptr, H3HIP_EINVAL, "bitmap rule without a bitmap");
  return H3HIP_OK;
}

// Small device arrays the rule kernel reads (global columns, landmark flags).
struct RuleScratch {
  uint8_t* d = nullptr;
  ~RuleScratch() {
    if (d) (void)hipFree(d);
  }
};

static int rule_to_device(const h3hip_mask_rule* r, RuleScratch& scratch, RuleDev& out,
                          hipStream_t stream) {
  const int32_t n_tiles = (r->seq_len + H3HIP_TILE - 1) / H3HIP_TILE;
  out = RuleDev{r->kind, r->seq_len, r->prefix_len, r->frames, r->height, r->width,
                r->frame_window, r->spatial_tile_h, r->spatial_tile_w, r->spatial_window,
                r->band, n_tiles, nullptr, nullptr};
  std::vector<uint8_t> host;
  size_t col_off = 0, lm_off = 0;
  if (r->kind == H3HIP_RULE_BAND) {
    col_off = host.size();
    host.resize(host.size() + n_tiles, 0);
    for (int32_t i = 0; i < r->n_global_cols; i++) host[col_off + r->global_cols[i]] = 1;
  }
  if ((r->kind == H3HIP_RULE_LOCAL || r->kind == H3HIP_RULE_AXIAL) && r->n_landmarks > 0) {
    lm_off = host.size();
    host.resize(host.size() + r->frames, 0);
    for (int32_t i = 0; i < r->n_landmarks; i++) host[lm_off + r->landmark_frames[i]] = 1;
  }
  if (host.empty()) return H3HIP_OK;
  H3_HIP_CHECK(hipMalloc(&scratch.d, host.size()));
  H3_HIP_CHECK(hipMemcpyAsync(scratch.d, host.data(), host.size(), hipMemcpyHostToDevice, stream));
  H3_HIP_CHECK(hipStreamSynchronize(stream));
  if (r->kind == H3HIP_RULE_BAND) out.col_global = scratch.d + col_off;
  if ((r->kind == H3HIP_RULE_LOCAL || r->kind == H3HIP_RULE_AXIAL) && r->n_landmarks > 0)
    out.frame_landmark = scratch.d + lm_off;
  return H3HIP_OK;
}

static int launch_mask(const h3hip_mask_rule* r, uint8_t* d_bitmap, hipStream_t stream,
                       RuleScratch& scratch) {
  const int32_t n_tiles = (r->seq_len + H3HIP_TILE - 1) / H3HIP_TILE;
  if (r->kind == H3HIP_RULE_BITMAP) {
    H3_HIP_CHECK(hipMemcpyAsync(d_bitmap, r->bitmap, (size_t)n_tiles * n_tiles,
                                hipMemcpyHostToDevice, stream));
    return H3HIP_OK;
  }
  RuleDev dev;
  int rc = rule_to_device(r, scratch, dev, stream);
  if (rc != H3HIP_OK) return rc;
  mask_rule_kernel<<<dim3(n_tiles, n_tiles), 256, 0, stream>>>(dev, d_bitmap);
  return check_launch("mask_rule_kernel");
}

// ---------------------------------------------- static scratch (no allocation)

// Device scratch for h3hip_mask_from_rule_noalloc: the rule's flag tables
// (BAND global columns, landmark frames) and the host lists they are built
// from, in one file-scope array per GPU that lives until the process ends.
// Layout: column flags [0, 32 KiB), frame flags [32 KiB, 64 KiB), the staged
// int32 list [64 KiB, 192 KiB).
constexpr int32_t kScratchFlags = 32768;   // max tile columns / frames
constexpr int32_t kScratchList = 32768;    // max global columns / landmarks
constexpr size_t kScratchBytes = 2 * kScratchFlags + 4 * (size_t)kScratchList;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// The scratch array's device address on each GPU, looked up once per device.
constexpr int kMaxDevices = 64;
static uint8_t* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_on_current_device(uint8_t** out) {
  int dev = 0;
  H3_HIP_CHECK(hipGetDevice(&dev));
  H3_REQUIRE(dev >= 0 && dev < kMaxDevices, H3HIP_EDEVICE, "device %d beyond %d", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    H3_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    H3_REQUIRE(p != nullptr, H3HIP_EHIP, "hipGetSymbolAddress returned NULL for the scratch");
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return H3HIP_OK;
}

// flags[0 .. n_flags) = 0, then flags[list[i]] = 1 for i < n_list (list
// entries are validated on the host). One workgroup; a fill kernel rather
// than a memset so the clear is an ordinary kernel node.
__global__ __launch_bounds__(256) void flags_from_list_kernel(uint8_t* flags, int32_t n_flags,
                                                              const int32_t* list,
                                                              int32_t n_list) {
  for (int32_t i = threadIdx.x; i < n_flags; i += 256) flags[i] = 0;
  __syncthreads();
  for (int32_t i = threadIdx.x; i < n_list; i += 256) flags[list[i]] = 1;
}

// The same with the list passed by value in the kernel arguments, so nothing
// is staged from host memory: the form h3hip_mask_from_rule_noalloc uses for
// short lists, which keeps it capturable into a HIP graph.
constexpr int32_t kArgList = 256;
struct ListArg {
  int32_t n;
  int32_t v[kArgList];
};
__global__ __launch_bounds__(256) void flags_from_arg_kernel(uint8_t* flags, int32_t n_flags,
                                                             ListArg list) {
  for (int32_t i = threadIdx.x; i < n_flags; i += 256) flags[i] = 0;
  __syncthreads();
  for (int32_t i = threadIdx.x; i < list.n; i += 256) flags[list.v[i]] = 1;
}

static int csr_on_device(const uint8_t* d_bitmap, int32_t nq, int32_t nk, int32_t* d_row_ptr,
                         hipStream_t stream, int64_t* nnz) {
  row_count_kernel<<<nq, 256, 0, stream>>>(d_bitmap, nk, d_row_ptr);
  int rc = check_launch("row_count_kernel");
  if (rc) return rc;
  scan_kernel<<<1, 256, 0, stream>>>(d_row_ptr, nq);
  rc = check_launch("scan_kernel");
  if (rc) return rc;
  int32_t last = 0;
  H3_HIP_CHECK(hipMemcpyAsync(&last, d_row_ptr + nq, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
  H3_HIP_CHECK(hipStreamSynchronize(stream));
  *nnz = last;
  return H3HIP_OK;
}

}  // namespace h3hip

using namespace h3hip;

extern "C" {

const char* h3hip_last_error(void) { return g_last_error.c_str(); }

const char* h3hip_version(void) { return "ch3hip 0.1 (gfx950)"; }

int h3hip_device_supported(int32_t device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int h3hip_mask_from_rule(const h3hip_mask_rule* rule, uint8_t* d_bitmap, void* stream) {
  int rc = validate_rule(rule);
  if (rc) return rc;
  H3_REQUIRE(d_bitmap != nullptr, H3HIP_EINVAL, "d_bitmap is NULL");
  RuleScratch scratch;
  rc = launch_mask(rule, d_bitmap, as_stream(stream), scratch);
  if (rc) return rc;
  // The scratch arrays are freed on return; make sure the kernel is done with them.
  if (scratch.d) H3_HIP_CHECK(hipStreamSynchronize(as_stream(stream)));
  return H3HIP_OK;
}

int h3hip_mask_from_rule_noalloc(const h3hip_mask_rule* rule, uint8_t* d_bitmap, void* stream) {
  int rc = validate_rule(rule);
  if (rc) return rc;
  H3_REQUIRE(d_bitmap != nullptr, H3HIP_EINVAL, "d_bitmap is NULL");
  hipStream_t st = as_stream(stream);
  // Under stream capture nothing may be staged from host memory: the copy would
  // re-read the caller's host array at every replay, and the synchronisation
  // that keeps that array alive is illegal while capturing.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  H3_HIP_CHECK(hipStreamIsCapturing(st, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  const int32_t n_tiles = (rule->seq_len + H3HIP_TILE - 1) / H3HIP_TILE;
  if (rule->kind == H3HIP_RULE_BITMAP) {
    H3_REQUIRE(!capturing, H3HIP_EINVAL,
               "a BITMAP rule copies the host bitmap and cannot run under stream capture");
    H3_HIP_CHECK(hipMemcpyAsync(d_bitmap, rule->bitmap, (size_t)n_tiles * n_tiles,
                                hipMemcpyHostToDevice, st));
    H3_HIP_CHECK(hipStreamSynchronize(st));
    return H3HIP_OK;
  }
  const bool band = rule->kind == H3HIP_RULE_BAND;
  const bool lattice = rule->kind == H3HIP_RULE_LOCAL || rule->kind == H3HIP_RULE_AXIAL;
  const int32_t n_list = band ? rule->n_global_cols : lattice ? rule->n_landmarks : 0;
  const int32_t n_flags = band ? n_tiles : lattice ? rule->frames : 0;
  const bool uses_scratch = n_list > 0 || band;
  H3_REQUIRE(!uses_scratch || n_flags <= kScratchFlags, H3HIP_EINVAL,
             "%d %s exceed the static scratch's %d flags", n_flags,
             band ? "tile columns" : "frames", kScratchFlags);
  H3_REQUIRE(n_list <= kScratchList, H3HIP_EINVAL,
             "%d listed %s exceed the static scratch's %d entries", n_list,
             band ? "global columns" : "landmarks", kScratchList);
  const bool by_value = n_list <= kArgList;
  H3_REQUIRE(by_value || !capturing, H3HIP_EINVAL,
             "%d listed %s exceed the %d that travel in kernel arguments; longer lists are "
             "staged from host memory and cannot run under stream capture",
             n_list, band ? "global columns" : "landmarks", kArgList);
  RuleDev dev{rule->kind, rule->seq_len, rule->prefix_len, rule->frames, rule->height,
              rule->width, rule->frame_window, rule->spatial_tile_h, rule->spatial_tile_w,
              rule->spatial_window, rule->band, n_tiles, nullptr, nullptr};
  bool staged = false;
  if (uses_scratch) {
    uint8_t* sp = nullptr;
    rc = scratch_on_current_device(&sp);
    if (rc) return rc;
    uint8_t* flags = band ? sp : sp + kScratchFlags;
    if (by_value) {
      ListArg arg{};
      arg.n = n_list;
      const int32_t* src = band ? rule->global_cols : rule->landmark_frames;
      for (int32_t i = 0; i < n_list; i++) arg.v[i] = src[i];
      flags_from_arg_kernel<<<1, 256, 0, st>>>(flags, n_flags, arg);
      rc = check_launch("flags_from_arg_kernel");
    } else {
      int32_t* list = reinterpret_cast<int32_t*>(sp + 2 * kScratchFlags);
      H3_HIP_CHECK(hipMemcpyAsync(list, band ? rule->global_cols : rule->landmark_frames,
                                  sizeof(int32_t) * n_list, hipMemcpyHostToDevice, st));
      staged = true;
      flags_from_list_kernel<<<1, 256, 0, st>>>(flags, n_flags, list, n_list);
      rc = check_launch("flags_from_list_kernel");
    }
    if (rc) return rc;
    if (band) dev.col_global = flags;
    else dev.frame_landmark = flags;
  }
  mask_rule_kernel<<<dim3(n_tiles, n_tiles), 256, 0, st>>>(dev, d_bitmap);
  rc = check_launch("mask_rule_kernel");
  if (rc) return rc;
  // A list staged from host memory must outlive the copy that consumes it.
  if (staged) H3_HIP_CHECK(hipStreamSynchronize(st));
  return H3HIP_OK;
}

int h3hip_tiles_from_mask(const uint8_t* d_bitmap, int32_t nq, int32_t nk, int32_t* d_row_ptr,
                          int32_t* d_col_idx, int64_t col_capacity, int64_t* nnz, void* stream) {
  H3_REQUIRE(d_bitmap && d_row_ptr && nnz, H3HIP_EINVAL, "NULL argument");
  H3_REQUIRE(nq > 0 && nk > 0, H3HIP_EINVAL, "nq and nk must be positive");
  hipStream_t s = as_stream(stream);
  int rc = csr_on_device(d_bitmap, nq, nk, d_row_ptr, s, nnz);
  if (rc) return rc;
  H3_REQUIRE(col_capacity >= *nnz, H3HIP_EINVAL, "col_capacity %lld < nnz %lld",
             (long long)col_capacity, (long long)*nnz);
  if (*nnz == 0) return H3HIP_OK;
  H3_REQUIRE(d_col_idx != nullptr, H3HIP_EINVAL, "d_col_idx is NULL");
  fill_kernel<<<nq, 256, 0, s>>>(d_bitmap, nk, d_row_ptr, d_col_idx);
  return check_launch("fill_kernel");
}

int h3hip_plan_create(const h3hip_mask_rule* rule, int32_t heads, const h3hip_policy* policy,
                      void* stream, h3hip_plan* out) {
  H3_REQUIRE(out != nullptr, H3HIP_EINVAL, "out is NULL");
  *out = nullptr;
  int rc = validate_rule(rule);
  if (rc) return rc;
  H3_REQUIRE(heads > 0 && heads < 32768, H3HIP_EINVAL, "heads %d out of range", heads);
  hipStream_t s = as_stream(stream);
  const int32_t n = (rule->seq_len + H3HIP_TILE - 1) / H3HIP_TILE;

  auto* p = new (std::nothrow) h3hip_plan_s();
  H3_REQUIRE(p != nullptr, H3HIP_ENOMEM, "plan allocation failed");
  p->seq_len = rule->seq_len;
  p->seq_pad = n * H3HIP_TILE;
  p->n_tiles = n;
  p->heads = heads;
  if (policy) p->policy = *policy;
  p->prefix_len = rule->prefix_len;
  p->kind = rule->kind;

  uint8_t* d_bitmap = nullptr;
  auto fail = [&](int code) {
    if (d_bitmap) (void)hipFree(d_bitmap);
    h3hip_plan_destroy(p);
    return code;
  };
  if (hipMalloc(&d_bitmap, (size_t)n * n) != hipSuccess ||
      hipMalloc(&p->d_row_ptr, sizeof(int32_t) * (n + 1)) != hipSuccess) {
    set_error("device allocation for the tile plan failed");
    return fail(H3HIP_ENOMEM);
  }
  RuleScratch scratch;
  rc = launch_mask(rule, d_bitmap, s, scratch);
  if (rc) return fail(rc);
  int64_t nnz = 0;
  rc = csr_on_device(d_bitmap, n, n, p->d_row_ptr, s, &nnz);
  if (rc) return fail(rc);
  p->nnz = nnz;
  if (hipMalloc(&p->d_col_idx, sizeof(int32_t) * std::max<int64_t>(nnz, 1)) != hipSuccess) {
    set_error("device allocation for %lld tile indices failed", (long long)nnz);
    return fail(H3HIP_ENOMEM);
  }
  if (nnz > 0) {
    fill_kernel<<<n, 256, 0, s>>>(d_bitmap, n, p->d_row_ptr, p->d_col_idx);
    rc = check_launch("fill_kernel");
    if (rc) return fail(rc);
  }
  p->row_ptr.resize(n + 1);
  p->col_idx.resize(nnz);
  if (hipMemcpyAsync(p->row_ptr.data(), p->d_row_ptr, sizeof(int32_t) * (n + 1),
                     hipMemcpyDeviceToHost, s) != hipSuccess ||
      (nnz > 0 && hipMemcpyAsync(p->col_idx.data(), p->d_col_idx, sizeof(int32_t) * nnz,
                                 hipMemcpyDeviceToHost, s) != hipSuccess) ||
      hipStreamSynchronize(s) != hipSuccess) {
    set_error("copying the tile lists back failed");
    return fail(H3HIP_EHIP);
  }
  (void)hipFree(d_bitmap);
  d_bitmap = nullptr;

  // One persistent attention workgroup per CU, a whole number per XCD.
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    set_error("querying the device's CU count failed");
    return fail(H3HIP_EHIP);
  }
  p->groups = std::max(8, cus / 8 * 8);
  rc = build_schedule(p->row_ptr, heads, p->groups, p->work_ptr, p->work);
  if (rc) return fail(rc);
  p->unit_desc.assign(p->work.size() * kUnitDescInts, 0);
  for (size_t u = 0; u < p->work.size(); u++) {
    const int32_t unit = p->work[u], qt = unit & 0xffff;
    const int32_t beg = p->row_ptr[qt], n = p->row_ptr[qt + 1] - beg;
    int32_t* d = &p->unit_desc[kUnitDescInts * u];
    d[0] = unit;
    d[1] = beg;
    d[2] = n;
    if (n > 0) {
      const int32_t* c = &p->col_idx[beg];
      d[3] = c[0];
      d[4] = c[n > 1 ? 1 : 0];
      d[5] = c[n > 2 ? 2 : n - 1];
      d[6] = (int64_t)c[n - 1] * 128 + 128 > p->seq_len ? 1 : 0;
    }
  }
  const size_t desc_bytes = sizeof(int32_t) * std::max<size_t>(p->unit_desc.size(), 1);
  if (hipMalloc(&p->d_work_ptr, sizeof(int32_t) * p->work_ptr.size()) != hipSuccess ||
      hipMalloc(&p->d_work, sizeof(int32_t) * std::max<size_t>(p->work.size(), 1)) != hipSuccess ||
      hipMalloc(&p->d_unit_desc, desc_bytes) != hipSuccess) {
    set_error("device allocation for the work list failed");
    return fail(H3HIP_ENOMEM);
  }
  if (hipMemcpyAsync(p->d_work_ptr, p->work_ptr.data(), sizeof(int32_t) * p->work_ptr.size(),
                     hipMemcpyHostToDevice, s) != hipSuccess ||
      (!p->work.empty() &&
       (hipMemcpyAsync(p->d_work, p->work.data(), sizeof(int32_t) * p->work.size(),
                       hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(p->d_unit_desc, p->unit_desc.data(),
                       sizeof(int32_t) * p->unit_desc.size(), hipMemcpyHostToDevice,
                       s) != hipSuccess)) ||
      hipStreamSynchronize(s) != hipSuccess) {
    set_error("uploading the work list failed");
    return fail(H3HIP_EHIP);
  }
  *out = p;
  return H3HIP_OK;
}

int h3hip_plan_destroy(h3hip_plan p) {
  if (!p) return H3HIP_OK;
  if (p->d_row_ptr) (void)hipFree(p->d_row_ptr);
  if (p->d_col_idx) (void)hipFree(p->d_col_idx);
  if (p->d_work) (void)hipFree(p->d_work);
  if (p->d_work_ptr) (void)hipFree(p->d_work_ptr);
  if (p->d_unit_desc) (void)hipFree(p->d_unit_desc);
  delete p;
  return H3HIP_OK;
}

int h3hip_plan_info(h3hip_plan p, int32_t* seq_len, int32_t* seq_pad, int32_t* n_tiles,
                    int64_t* nnz, int32_t* heads) {
  H3_REQUIRE(p != nullptr, H3HIP_EINVAL, "plan is NULL");
  if (seq_len) *seq_len = p->seq_len;
  if (seq_pad) *seq_pad = p->seq_pad;
  if (n_tiles) *n_tiles = p->n_tiles;
  if (nnz) *nnz = p->nnz;
  if (heads) *heads = p->heads;
  return H3HIP_OK;
}

int h3hip_plan_tiles(h3hip_plan p, int32_t* row_ptr, int32_t* col_idx) {
  H3_REQUIRE(p != nullptr, H3HIP_EINVAL, "plan is NULL");
  if (row_ptr) std::memcpy(row_ptr, p->row_ptr.data(), sizeof(int32_t) * p->row_ptr.size());
  if (col_idx && p->nnz > 0) std::memcpy(col_idx, p->col_idx.data(), sizeof(int32_t) * p->nnz);
  return H3HIP_OK;
}

double h3hip_plan_density(h3hip_plan p) {
  if (!p || p->n_tiles == 0) return 0.0;
  return (double)p->nnz / ((double)p->n_tiles * (double)p->n_tiles);
}

}  // extern "C"
