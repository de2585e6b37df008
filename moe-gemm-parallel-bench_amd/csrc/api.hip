// C ABI of libmoegemm: the native boundary under kernels/grouped_gemm.py and kernels/matmul.py.
//
// Every entry point takes plain device pointers, integer sizes and a hipStream_t passed as void*.
// Nothing here allocates, synchronizes or copies: a call is one kernel launch on the caller's
// stream (capturable in a HIP graph) or an error code with a message in moegemm_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/moegemm.h"
#include "registry.h"

using namespace moegemm;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

const KernelEntry* table_for(int dtype, int* count) {
  switch (dtype) {
    case DT_BF16: *count = kNumBf16; return kEntriesBf16;
    case DT_F16: *count = kNumF16; return kEntriesF16;
    case DT_F32: *count = kNumF32; return kEntriesF32;
    default: *count = 0; return nullptr;
  }
}

const KernelEntry* find_entry(int dtype, int bm, int bn, int bk, int warps, int stages) {
  int count = 0;
  const KernelEntry* t = table_for(dtype, &count);
  for (int i = 0; i < count; ++i) {
    const KernelEntry& e = t[i];
    if (e.block_m == bm && e.block_n == bn && e.block_k == bk && e.num_warps == warps && e.num_stages == stages)
      return &e;
  }
  return nullptr;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int check_common(int dtype, int input_precision, int group_size_m, const KernelEntry** entry, int bm, int bn, int bk,
                 int warps, int stages) {
  if (dtype != DT_F16 && dtype != DT_BF16 && dtype != DT_F32)
    return fail(MOEGEMM_ERR_INVALID, "unsupported dtype code %d", dtype);
  if (input_precision != MOEGEMM_PRECISION_IEEE && input_precision != MOEGEMM_PRECISION_TF32)
    return fail(MOEGEMM_ERR_INVALID, "unsupported input precision code %d", input_precision);
  if (input_precision == MOEGEMM_PRECISION_TF32 && dtype != DT_F32)
    return fail(MOEGEMM_ERR_INVALID, "tf32 input precision requires fp32 operands");
  if (group_size_m <= 0) return fail(MOEGEMM_ERR_INVALID, "group_size_m must be positive (got %d)", group_size_m);
  *entry = find_entry(dtype, bm, bn, bk, warps, stages);
  if (!*entry)
    return fail(MOEGEMM_ERR_NO_KERNEL,
                "no compiled kernel for dtype=%d block_m=%d block_n=%d block_k=%d num_warps=%d num_stages=%d", dtype, bm,
                bn, bk, warps, stages);
  return MOEGEMM_OK;
}

int launch(const KernelEntry* e, KParams& p, int grid, bool vector_layout, int32_t b_stream, void* stream) {
  if (b_stream != 0 && b_stream != 1) return fail(MOEGEMM_ERR_INVALID, "b_stream must be 0 or 1 (got %d)", b_stream);
  p.b_stream = b_stream;
  LaunchFn fn = (vector_layout && e->launch_fast) ? e->launch_fast : e->launch_general;
  if (p.sk_tiles > 0) {  // stream-K tail: the fast path's stream-K kernel (the callers checked the layout)
    if (!vector_layout || !e->launch_fast_streamk)
      return fail(MOEGEMM_ERR_INVALID, "stream-K needs fp16/bf16 operands in the vector layout");
    fn = e->launch_fast_streamk;
  } else if (p.splits > 1) {  // split-K units: the fast path's split kernel (the callers checked the layout)
    if (!vector_layout || !e->launch_fast_split)
      return fail(MOEGEMM_ERR_INVALID, "split-K needs fp16/bf16 operands in the vector layout");
    fn = e->launch_fast_split;
  }
  hipError_t err = fn(p, grid, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(MOEGEMM_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return MOEGEMM_OK;
}

// Split-K workspace: a fixed-size area of int32 tile counters at offset 0, then the fp32 partials
// [tiles][splits][BM*BN].  The counter area has the same size whatever the launch, so the partials
// of one launch never overlap the counters of another launch that shares the workspace (a counter
// left non-zero by a stray partial would never see its tile's last unit, and the tile would go
// unstored); counters are only ever written as counters, and every launch leaves them zero.
constexpr int64_t kSplitCounterBytes = 256 * 1024;
constexpr int64_t kSplitMaxTiles = kSplitCounterBytes / 4;

int64_t splitk_bytes(int64_t tiles, int64_t splits, int64_t block_m, int64_t block_n) {
  return kSplitCounterBytes + tiles * splits * block_m * block_n * 4;
}

// Polls a split-K unit makes of its tile's counter while it waits for the tile's other units (see
// FastTile::split_store).  MOEGEMM_SPLIT_POLLS overrides the default of 16 (0 = never wait); tests
// set it to force the path where units stop waiting.
int32_t split_polls() {
  const char* env = std::getenv("MOEGEMM_SPLIT_POLLS");
  if (!env || !*env) return 16;
  const long v = std::strtol(env, nullptr, 10);
  return v < 0 ? 0 : v > 4096 ? 4096 : (int32_t)v;
}

// The K range of each split (whole K slices) and the split count that runs: trailing splits that
// would be empty are dropped.  Shared by setup_splits and the no-allocation size check.
void split_plan(int64_t k, int64_t splits, int64_t block_k, int64_t* chunk, int64_t* effective) {
  *chunk = cdiv(cdiv(k, splits), block_k) * block_k;
  *effective = cdiv(k, *chunk);
}

int setup_splits(KParams& p, int64_t tiles, int32_t k, int32_t splits, int32_t block_m, int32_t block_n,
                 int32_t block_k, void* workspace, int64_t workspace_bytes) {
  if (splits < 1 || splits > 64) return fail(MOEGEMM_ERR_INVALID, "splits must be in [1, 64] (got %d)", splits);
  int64_t chunk = 0, effective = 0;
  split_plan(k, splits, block_k, &chunk, &effective);
  if (tiles * effective > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "split-K unit count exceeds int32");
  if (effective > 1) {
    if (tiles > kSplitMaxTiles)
      return fail(MOEGEMM_ERR_INVALID, "split-K supports at most %lld output tiles (got %lld)",
                  (long long)kSplitMaxTiles, (long long)tiles);
    const int64_t need = splitk_bytes(tiles, effective, block_m, block_n);
    if (!workspace || workspace_bytes < need)
      return fail(MOEGEMM_ERR_INVALID, "split-K workspace of %lld bytes is smaller than the %lld needed",
                  (long long)workspace_bytes, (long long)need);
    if (reinterpret_cast<uintptr_t>(workspace) & 255)
      return fail(MOEGEMM_ERR_INVALID, "split-K workspace must be 256-byte aligned");
    p.counters = static_cast<int32_t*>(workspace);
    p.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kSplitCounterBytes);
  }
  p.splits = (int32_t)effective;
  p.k_chunk = (int32_t)chunk;
  p.split_polls = split_polls();
  p.total_tiles = (int32_t)tiles;
  return MOEGEMM_OK;
}

// Stream-K tail workspace: the split-K counter area, then grid + tail_tiles fp32 partial slots
// (piece (run v, tail tile j) writes slot v + j; see streamk_units in gemm_kernel.h).
int64_t streamk_bytes(int64_t tail_tiles, int64_t grid, int64_t block_m, int64_t block_n) {
  return kSplitCounterBytes + (grid + tail_tiles) * block_m * block_n * 4;
}

// Checks a stream-K plan and fills the launch fields: total_tiles tiles, the last tail_tiles of
// them cut into `grid` runs of K slices.  A tail tile is cut into at most ceil(KT / floor(I / W))
// + 1 pieces (I = tail_tiles * KT slices over W = grid runs); at most 64 are allowed, as for
// split-K, so every run holds at least about KT / 63 slices.
int setup_streamk(KParams& p, int64_t tiles, int32_t k, int32_t tail_tiles, int32_t grid, int32_t block_m,
                  int32_t block_n, int32_t block_k, void* workspace, int64_t workspace_bytes) {
  if (grid <= 0) return fail(MOEGEMM_ERR_INVALID, "stream-K needs a positive persistent grid (got %d)", grid);
  if (tail_tiles < 1 || tail_tiles > tiles)
    return fail(MOEGEMM_ERR_INVALID, "stream-K tail of %d tiles is outside [1, %lld]", tail_tiles, (long long)tiles);
  if (tail_tiles > kSplitMaxTiles)
    return fail(MOEGEMM_ERR_INVALID, "stream-K supports tails of at most %lld tiles (got %d)",
                (long long)kSplitMaxTiles, tail_tiles);
  const int64_t kt = cdiv(k, block_k);
  const int64_t per_run = (int64_t)tail_tiles * kt / grid;
  if (per_run < 1 || cdiv(kt, per_run) + 1 > 64)
    return fail(MOEGEMM_ERR_INVALID,
                "stream-K tail too thin: %d tiles of %lld K slices over %d runs cut a tile into more than 64 pieces",
                tail_tiles, (long long)kt, grid);
  const int64_t need = streamk_bytes(tail_tiles, grid, block_m, block_n);
  if (!workspace || workspace_bytes < need)
    return fail(MOEGEMM_ERR_INVALID, "stream-K workspace of %lld bytes is smaller than the %lld needed",
                (long long)workspace_bytes, (long long)need);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(MOEGEMM_ERR_INVALID, "stream-K workspace must be 256-byte aligned");
  p.counters = static_cast<int32_t*>(workspace);
  p.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kSplitCounterBytes);
  p.splits = 1;
  p.k_chunk = k;
  p.split_polls = 0;
  p.sk_tiles = tail_tiles;
  p.total_tiles = (int32_t)tiles;
  return MOEGEMM_OK;
}

// Static split-K scratch of the no-allocation entry point: the same layout as a caller workspace
// (counters, then partials).  Each GPU holds its own copy from module load until the process ends.
// Host code never uses the array's name as an address (in host code it is a stand-in, not device
// memory): each device's address comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address is passed to kernels.
static __device__ __align__(256) char scratch[MOEGEMM_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

__global__ void clear_counters(int32_t* counters, int32_t words) {
  for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) counters[i] = 0;
}

// Address of the current device's scratch area.  The first call on a device looks it up and
// clears the counter area with a kernel on `stream` (so a first call inside graph capture records
// a kernel, not a memset); every later launch leaves the counters zero again.
int device_scratch(void* stream, void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(MOEGEMM_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(MOEGEMM_ERR_INVALID, "device index %d is beyond the %d devices the library tracks", device,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_address[device]) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !address)
      return fail(MOEGEMM_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(err));
    const int32_t words = (int32_t)(kSplitCounterBytes / 4);
    hipLaunchKernelGGL(clear_counters, dim3(64), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<int32_t*>(address), words);
    err = hipGetLastError();
    if (err != hipSuccess)
      return fail(MOEGEMM_ERR_LAUNCH, "clearing the scratch counters failed: %s", hipGetErrorString(err));
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return MOEGEMM_OK;
}

// Byte-range limits of the LDS-DMA kernels' 32-bit buffer offsets (see gemm_fast.h): A and C are
// addressed through one resource per tile spanning at most kPanelRows rows, B through one
// resource from the tile's first column to the end of the matrix.
constexpr int64_t kTwoGiB = int64_t(1) << 31;
constexpr int64_t kPanelRows = 256;  // the largest block_m of the menu

bool panels_fit(int64_t k, int64_t sam, int64_t sbk, int64_t scm) {
  return kPanelRows * sam * 2 < kTwoGiB && kPanelRows * scm * 2 < kTwoGiB && k * sbk * 2 < kTwoGiB;
}

// Preconditions of the LDS-DMA fast path for one problem (see gemm_fast.h).
bool vector_layout_ok(const void* a, const void* b, const void* c, int64_t m, int64_t n, int64_t k, int64_t sam,
                      int64_t sak, int64_t sbk, int64_t sbn, int64_t scm, int64_t scn, int dtype) {
  (void)m;  // A and C may be any number of rows: their resources are per tile
  if (dtype != DT_BF16 && dtype != DT_F16) return false;
  if (sak != 1 || sbn != 1 || scn != 1) return false;
  if (k % 8 || n % 8 || sam % 8 || sbk % 8 || scm % 4 || sam < k || sbk < n || scm < n) return false;
  if ((reinterpret_cast<uintptr_t>(a) & 15) || (reinterpret_cast<uintptr_t>(b) & 15) ||
      (reinterpret_cast<uintptr_t>(c) & 7))
    return false;
  return panels_fit(k, sam, sbk, scm);
}

}  // namespace

extern "C" {

int moegemm_abi_version(void) { return MOEGEMM_ABI_VERSION; }

const char* moegemm_last_error(void) { return g_last_error.c_str(); }

int moegemm_kernel_count(int dtype) {
  int count = 0;
  table_for(dtype, &count);
  return count;
}

int moegemm_kernel_info(int dtype, int index, int32_t* out7) {
  int count = 0;
  const KernelEntry* t = table_for(dtype, &count);
  if (!t || index < 0 || index >= count || !out7)
    return fail(MOEGEMM_ERR_INVALID, "kernel index %d out of range for dtype %d", index, dtype);
  const KernelEntry& e = t[index];
  out7[0] = e.block_m;
  out7[1] = e.block_n;
  out7[2] = e.block_k;
  out7[3] = e.num_warps;
  out7[4] = e.num_stages;
  out7[5] = e.lds_bytes;
  out7[6] = e.waves_m;
  return MOEGEMM_OK;
}

}  // extern "C"

namespace {

// Work-stealing queue: MOEGEMM_QUEUE_BYTES of int32 counters, zero before the first launch (each
// launch leaves them zero).  Null keeps the static schedule.
int set_queue(KParams& p, void* queue) {
  if (queue && (reinterpret_cast<uintptr_t>(queue) & 255))
    return fail(MOEGEMM_ERR_INVALID, "the tile queue must be 256-byte aligned");
  static_assert(kQueueSlots * kQueueStride * 4 <= MOEGEMM_QUEUE_BYTES, "queue counters fit the documented size");
  p.queue = static_cast<int32_t*>(queue);
  return MOEGEMM_OK;
}

int grouped_impl(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs, const int32_t* dims,
                 const int64_t* strides, int32_t problem_count, int32_t m, int32_t n, int32_t k, int32_t homogeneous,
                 int32_t total_tiles, int32_t dtype, int32_t input_precision, int32_t block_m, int32_t block_n,
                 int32_t block_k, int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t grid_size,
                 int32_t vector_layout, bool swiglu, void* queue, int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, input_precision, group_size_m, &e, block_m, block_n, block_k, num_warps, num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (swiglu) {
    if (dtype != DT_BF16 && dtype != DT_F16)
      return fail(MOEGEMM_ERR_INVALID, "the SwiGLU epilogue needs fp16 or bf16 operands");
    if (!vector_layout)
      return fail(MOEGEMM_ERR_INVALID, "the SwiGLU epilogue needs the vector layout (LDS-DMA kernel)");
    if (!e->swiglu_ok)
      return fail(MOEGEMM_ERR_INVALID,
                  "tile %dx%dx%d with %d waves cannot pair gate and up fragments (odd fragments per wave)",
                  block_m, block_n, block_k, num_warps);
    if (homogeneous && n % 16)
      return fail(MOEGEMM_ERR_INVALID, "packed Gate+Up width must be a multiple of 16 (got %d)", n);
  }
  if (problem_count <= 0) return fail(MOEGEMM_ERR_INVALID, "problem_count must be positive (got %d)", problem_count);
  if (!a_ptrs || !b_ptrs || !c_ptrs) return fail(MOEGEMM_ERR_INVALID, "pointer tables must be non-null");
  if (total_tiles < 0) return fail(MOEGEMM_ERR_INVALID, "total_tiles must be non-negative");
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.a_ptrs = a_ptrs;
  p.b_ptrs = b_ptrs;
  p.c_ptrs = c_ptrs;
  p.G = problem_count;
  p.group_m = group_size_m;
  p.tf32 = input_precision == MOEGEMM_PRECISION_TF32;
  p.swiglu = swiglu ? 1 : 0;
  if (homogeneous) {
    if (m <= 0 || n <= 0 || k <= 0)
      return fail(MOEGEMM_ERR_INVALID, "homogeneous shape must be positive (m=%d n=%d k=%d)", m, n, k);
    int64_t tiles = (int64_t)problem_count * cdiv(m, block_m) * cdiv(n, block_n);
    if (tiles > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "tile count %lld exceeds int32", (long long)tiles);
    p.mode = MODE_HOMOGENEOUS;
    p.M = m;
    p.N = n;
    p.K = k;
    p.total_tiles = (int32_t)tiles;
  } else {
    if (!dims || !strides) return fail(MOEGEMM_ERR_INVALID, "generic groups need dims and strides tables");
    p.mode = MODE_GENERIC;
    p.dims = dims;
    p.strides = strides;
    p.total_tiles = total_tiles;
  }
  rc = set_queue(p, queue);
  if (rc != MOEGEMM_OK) return rc;
  if (p.total_tiles == 0) return MOEGEMM_OK;
  int grid = grid_size <= 0 ? p.total_tiles : (grid_size < p.total_tiles ? grid_size : p.total_tiles);
  return launch(e, p, grid, vector_layout != 0, b_stream, stream);
}

}  // namespace

extern "C" {

int moegemm_grouped_gemm(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs, const int32_t* dims,
                         const int64_t* strides, int32_t problem_count, int32_t m, int32_t n, int32_t k,
                         int32_t homogeneous, int32_t total_tiles, int32_t dtype, int32_t input_precision,
                         int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m, int32_t num_warps,
                         int32_t num_stages, int32_t grid_size, int32_t vector_layout, int32_t b_stream, void* stream) {
  return grouped_impl(a_ptrs, b_ptrs, c_ptrs, dims, strides, problem_count, m, n, k, homogeneous, total_tiles, dtype,
                      input_precision, block_m, block_n, block_k, group_size_m, num_warps, num_stages, grid_size,
                      vector_layout, false, nullptr, b_stream, stream);
}

int moegemm_grouped_gemm_stealing(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                                  const int32_t* dims, const int64_t* strides, int32_t problem_count, int32_t m,
                                  int32_t n, int32_t k, int32_t homogeneous, int32_t total_tiles, int32_t dtype,
                                  int32_t input_precision, int32_t block_m, int32_t block_n, int32_t block_k,
                                  int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t grid_size,
                                  int32_t vector_layout, void* queue, int32_t b_stream, void* stream) {
  if (!queue) return fail(MOEGEMM_ERR_INVALID, "the work-stealing launch needs a tile queue");
  return grouped_impl(a_ptrs, b_ptrs, c_ptrs, dims, strides, problem_count, m, n, k, homogeneous, total_tiles, dtype,
                      input_precision, block_m, block_n, block_k, group_size_m, num_warps, num_stages, grid_size,
                      vector_layout, false, queue, b_stream, stream);
}

int moegemm_grouped_gemm_swiglu(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* h_ptrs,
                                const int32_t* dims, const int64_t* strides, int32_t problem_count, int32_t m,
                                int32_t n, int32_t k, int32_t homogeneous, int32_t total_tiles, int32_t dtype,
                                int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                                int32_t num_warps, int32_t num_stages, int32_t grid_size, int32_t vector_layout,
                                int32_t b_stream, void* stream) {
  return grouped_impl(a_ptrs, b_ptrs, h_ptrs, dims, strides, problem_count, m, n, k, homogeneous, total_tiles, dtype,
                      MOEGEMM_PRECISION_IEEE, block_m, block_n, block_k, group_size_m, num_warps, num_stages,
                      grid_size, vector_layout, true, nullptr, b_stream, stream);
}

int moegemm_splitk_workspace_bytes(int32_t tiles, int32_t splits, int32_t block_m, int32_t block_n, int64_t* bytes) {
  if (tiles < 0 || splits < 1 || block_m <= 0 || block_n <= 0 || !bytes)
    return fail(MOEGEMM_ERR_INVALID, "split-K workspace query needs tiles >= 0, splits >= 1 and a tile shape");
  *bytes = splitk_bytes(tiles, splits, block_m, block_n);
  return MOEGEMM_OK;
}

static int matmul_splitk_impl(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k, int64_t stride_am,
                          int64_t stride_ak, int64_t stride_bk, int64_t stride_bn, int64_t stride_cm,
                          int64_t stride_cn, int32_t dtype, int32_t block_m, int32_t block_n, int32_t block_k,
                          int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t splits,
                          int32_t grid_size, void* workspace, int64_t workspace_bytes, int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, MOEGEMM_PRECISION_IEEE, group_size_m, &e, block_m, block_n, block_k, num_warps,
                        num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (!a || !b || !c) return fail(MOEGEMM_ERR_INVALID, "matrix pointers must be non-null");
  if (m <= 0 || n <= 0 || k <= 0) return fail(MOEGEMM_ERR_INVALID, "shape must be positive (m=%d n=%d k=%d)", m, n, k);
  if (!vector_layout_ok(a, b, c, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn, dtype) ||
      !e->launch_fast)
    return fail(MOEGEMM_ERR_INVALID, "split-K needs fp16/bf16 operands in the vector layout");
  const int64_t tiles = cdiv(m, block_m) * cdiv(n, block_n);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_SINGLE;
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = m;
  p.N = n;
  p.K = k;
  p.sam = stride_am;
  p.sak = stride_ak;
  p.sbk = stride_bk;
  p.sbn = stride_bn;
  p.scm = stride_cm;
  p.scn = stride_cn;
  p.G = 1;
  p.group_m = group_size_m;
  rc = setup_splits(p, tiles, k, splits, block_m, block_n, block_k, workspace, workspace_bytes);
  if (rc != MOEGEMM_OK) return rc;
  const int64_t units = (int64_t)p.total_tiles * p.splits;
  const int grid = grid_size <= 0 || grid_size > units ? (int)units : grid_size;
  return launch(e, p, grid, true, b_stream, stream);
}

int moegemm_matmul_splitk(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k, int64_t stride_am,
                          int64_t stride_ak, int64_t stride_bk, int64_t stride_bn, int64_t stride_cm,
                          int64_t stride_cn, int32_t dtype, int32_t block_m, int32_t block_n, int32_t block_k,
                          int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t splits,
                          int32_t grid_size, void* workspace, int64_t workspace_bytes, int32_t b_stream, void* stream) {
  return matmul_splitk_impl(a, b, c, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn, dtype,
                            block_m, block_n, block_k, group_size_m, num_warps, num_stages, splits, grid_size,
                            workspace, workspace_bytes, b_stream, stream);
}

int moegemm_matmul_splitk_noalloc(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k,
                                  int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                                  int64_t stride_cm, int64_t stride_cn, int32_t dtype, int32_t block_m,
                                  int32_t block_n, int32_t block_k, int32_t group_size_m, int32_t num_warps,
                                  int32_t num_stages, int32_t splits, int32_t grid_size,
                                  int32_t b_stream, void* stream) {
  // The split count that will run decides the bytes needed (split_plan, as setup_splits computes
  // it); a launch whose partials would not fit the static area is rejected before anything runs.
  // Other bad arguments are left to matmul_splitk_impl's checks.
  if (splits >= 1 && splits <= 64 && block_m > 0 && block_n > 0 && block_k > 0 && m > 0 && n > 0 && k > 0) {
    int64_t chunk = 0, effective = 0;
    split_plan(k, splits, block_k, &chunk, &effective);
    const int64_t need = splitk_bytes(cdiv(m, block_m) * cdiv(n, block_n), effective, block_m, block_n);
    if (effective > 1 && need > MOEGEMM_NOALLOC_SCRATCH_BYTES)
      return fail(MOEGEMM_ERR_INVALID,
                  "split-K launch needs %lld bytes of scratch, beyond the %lld-byte static area of the "
                  "no-allocation entry point; use moegemm_matmul_splitk with a workspace",
                  (long long)need, (long long)MOEGEMM_NOALLOC_SCRATCH_BYTES);
  }
  void* area = nullptr;
  int rc = device_scratch(stream, &area);
  if (rc != MOEGEMM_OK) return rc;
  return matmul_splitk_impl(a, b, c, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn, dtype,
                            block_m, block_n, block_k, group_size_m, num_warps, num_stages, splits, grid_size, area,
                            MOEGEMM_NOALLOC_SCRATCH_BYTES, b_stream, stream);
}

int moegemm_grouped_gemm_splitk(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                                int32_t problem_count, int32_t m, int32_t n, int32_t k, int32_t dtype,
                                int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                                int32_t num_warps, int32_t num_stages, int32_t splits, int32_t grid_size,
                                int32_t vector_layout, void* workspace, int64_t workspace_bytes,
                                int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, MOEGEMM_PRECISION_IEEE, group_size_m, &e, block_m, block_n, block_k, num_warps,
                        num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (problem_count <= 0) return fail(MOEGEMM_ERR_INVALID, "problem_count must be positive (got %d)", problem_count);
  if (!a_ptrs || !b_ptrs || !c_ptrs) return fail(MOEGEMM_ERR_INVALID, "pointer tables must be non-null");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail(MOEGEMM_ERR_INVALID, "homogeneous shape must be positive (m=%d n=%d k=%d)", m, n, k);
  if (!vector_layout || !e->launch_fast)
    return fail(MOEGEMM_ERR_INVALID, "split-K needs fp16/bf16 operands in the vector layout");
  const int64_t tiles = (int64_t)problem_count * cdiv(m, block_m) * cdiv(n, block_n);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_HOMOGENEOUS;
  p.a_ptrs = a_ptrs;
  p.b_ptrs = b_ptrs;
  p.c_ptrs = c_ptrs;
  p.G = problem_count;
  p.M = m;
  p.N = n;
  p.K = k;
  p.group_m = group_size_m;
  rc = setup_splits(p, tiles, k, splits, block_m, block_n, block_k, workspace, workspace_bytes);
  if (rc != MOEGEMM_OK) return rc;
  const int64_t units = (int64_t)p.total_tiles * p.splits;
  const int grid = grid_size <= 0 || grid_size > units ? (int)units : grid_size;
  return launch(e, p, grid, true, b_stream, stream);
}

int moegemm_streamk_workspace_bytes(int32_t tail_tiles, int32_t grid_size, int32_t block_m, int32_t block_n,
                                    int64_t* bytes) {
  if (tail_tiles < 0 || grid_size < 1 || block_m <= 0 || block_n <= 0 || !bytes)
    return fail(MOEGEMM_ERR_INVALID, "stream-K workspace query needs tail_tiles >= 0, grid_size >= 1 and a tile shape");
  *bytes = streamk_bytes(tail_tiles, grid_size, block_m, block_n);
  return MOEGEMM_OK;
}

int moegemm_matmul_streamk(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k, int64_t stride_am,
                           int64_t stride_ak, int64_t stride_bk, int64_t stride_bn, int64_t stride_cm,
                           int64_t stride_cn, int32_t dtype, int32_t block_m, int32_t block_n, int32_t block_k,
                           int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t tail_tiles,
                           int32_t grid_size, void* workspace, int64_t workspace_bytes,
                           int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, MOEGEMM_PRECISION_IEEE, group_size_m, &e, block_m, block_n, block_k, num_warps,
                        num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (!a || !b || !c) return fail(MOEGEMM_ERR_INVALID, "matrix pointers must be non-null");
  if (m <= 0 || n <= 0 || k <= 0) return fail(MOEGEMM_ERR_INVALID, "shape must be positive (m=%d n=%d k=%d)", m, n, k);
  if (!vector_layout_ok(a, b, c, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn, dtype) ||
      !e->launch_fast)
    return fail(MOEGEMM_ERR_INVALID, "stream-K needs fp16/bf16 operands in the vector layout");
  const int64_t tiles = cdiv(m, block_m) * cdiv(n, block_n);
  if (tiles > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "tile count %lld exceeds int32", (long long)tiles);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_SINGLE;
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = m;
  p.N = n;
  p.K = k;
  p.sam = stride_am;
  p.sak = stride_ak;
  p.sbk = stride_bk;
  p.sbn = stride_bn;
  p.scm = stride_cm;
  p.scn = stride_cn;
  p.G = 1;
  p.group_m = group_size_m;
  rc = setup_streamk(p, tiles, k, tail_tiles, grid_size, block_m, block_n, block_k, workspace, workspace_bytes);
  if (rc != MOEGEMM_OK) return rc;
  return launch(e, p, grid_size, true, b_stream, stream);
}

int moegemm_grouped_gemm_streamk(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                                 int32_t problem_count, int32_t m, int32_t n, int32_t k, int32_t dtype,
                                 int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                                 int32_t num_warps, int32_t num_stages, int32_t tail_tiles, int32_t grid_size,
                                 int32_t vector_layout, void* workspace, int64_t workspace_bytes,
                                 int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, MOEGEMM_PRECISION_IEEE, group_size_m, &e, block_m, block_n, block_k, num_warps,
                        num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (problem_count <= 0) return fail(MOEGEMM_ERR_INVALID, "problem_count must be positive (got %d)", problem_count);
  if (!a_ptrs || !b_ptrs || !c_ptrs) return fail(MOEGEMM_ERR_INVALID, "pointer tables must be non-null");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail(MOEGEMM_ERR_INVALID, "homogeneous shape must be positive (m=%d n=%d k=%d)", m, n, k);
  if (!vector_layout || !e->launch_fast)
    return fail(MOEGEMM_ERR_INVALID, "stream-K needs fp16/bf16 operands in the vector layout");
  const int64_t tiles = (int64_t)problem_count * cdiv(m, block_m) * cdiv(n, block_n);
  if (tiles > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "tile count %lld exceeds int32", (long long)tiles);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_HOMOGENEOUS;
  p.a_ptrs = a_ptrs;
  p.b_ptrs = b_ptrs;
  p.c_ptrs = c_ptrs;
  p.G = problem_count;
  p.M = m;
  p.N = n;
  p.K = k;
  p.group_m = group_size_m;
  rc = setup_streamk(p, tiles, k, tail_tiles, grid_size, block_m, block_n, block_k, workspace, workspace_bytes);
  if (rc != MOEGEMM_OK) return rc;
  return launch(e, p, grid_size, true, b_stream, stream);
}

int moegemm_kernel_swiglu(int dtype, int index) {
  int count = 0;
  const KernelEntry* t = table_for(dtype, &count);
  if (!t || index < 0 || index >= count)
    return fail(MOEGEMM_ERR_INVALID, "kernel index %d out of range for dtype %d", index, dtype);
  return t[index].swiglu_ok;
}

// `swiglu`: B holds [gate | up] (n = 2F columns) and C is H [rows, F] (row stride stride_cm).
static int offsets_impl(const void* a, const void* b, void* c, const int32_t* offs, int32_t group_count, int32_t rows,
                        int32_t n, int32_t k, int64_t stride_am, int64_t stride_bg, int64_t stride_bk,
                        int64_t stride_cm, int32_t dtype, int32_t input_precision, int32_t block_m, int32_t block_n,
                        int32_t block_k, int32_t group_size_m, int32_t num_warps, int32_t num_stages,
                        int32_t grid_size, bool swiglu, void* queue, int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, input_precision, group_size_m, &e, block_m, block_n, block_k, num_warps, num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (!a || !b || !c || !offs) return fail(MOEGEMM_ERR_INVALID, "matrix and offsets pointers must be non-null");
  if (group_count <= 0) return fail(MOEGEMM_ERR_INVALID, "group_count must be positive (got %d)", group_count);
  if (rows < 0 || n <= 0 || k <= 0)
    return fail(MOEGEMM_ERR_INVALID, "shape must have rows >= 0 and positive n, k (rows=%d n=%d k=%d)", rows, n, k);
  const int64_t out_cols = swiglu ? n / 2 : n;
  if (swiglu) {
    if (dtype != DT_BF16 && dtype != DT_F16)
      return fail(MOEGEMM_ERR_INVALID, "the SwiGLU epilogue needs fp16 or bf16 operands");
    if (!e->swiglu_ok)
      return fail(MOEGEMM_ERR_INVALID,
                  "tile %dx%dx%d with %d waves cannot pair gate and up fragments (odd fragments per wave)",
                  block_m, block_n, block_k, num_warps);
    if (n % 16) return fail(MOEGEMM_ERR_INVALID, "packed Gate+Up width must be a multiple of 16 (got %d)", n);
  }
  if (stride_am < k || stride_bk < n || stride_cm < out_cols || stride_bg < (int64_t)k * stride_bk)
    return fail(MOEGEMM_ERR_INVALID,
                "strides overlap rows or groups (stride_am=%lld stride_bk=%lld stride_bg=%lld stride_cm=%lld)",
                (long long)stride_am, (long long)stride_bk, (long long)stride_bg, (long long)stride_cm);
  if (rows == 0) return MOEGEMM_OK;
  // Upper bound on the tile count: every group adds at most one partial M tile.
  const int64_t m_tiles = std::min<int64_t>(rows / block_m + group_count, (int64_t)group_count * cdiv(rows, block_m));
  const int64_t tiles = m_tiles * cdiv(n, block_n);
  if (tiles > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "tile bound %lld exceeds int32", (long long)tiles);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_OFFSETS;
  p.a = a;
  p.b = b;
  p.c = c;
  p.offs = offs;
  p.G = group_count;
  p.rows = rows;
  p.N = n;
  p.K = k;
  p.sam = stride_am;
  p.sbk = stride_bk;
  p.sbg = stride_bg;
  p.scm = stride_cm;
  p.group_m = group_size_m;
  p.tf32 = input_precision == MOEGEMM_PRECISION_TF32;
  p.total_tiles = (int32_t)tiles;
  p.swiglu = swiglu ? 1 : 0;
  const int grid = grid_size <= 0 ? p.total_tiles : (grid_size < p.total_tiles ? grid_size : p.total_tiles);
  // Every group shares the strides, so one check covers all of them; the A and C resources of a
  // tile span at most block_m rows, each group's B resource one [k, n] panel.
  const bool vec = (dtype == DT_BF16 || dtype == DT_F16) && k % 8 == 0 && n % 8 == 0 && stride_am % 8 == 0 &&
                   stride_bk % 8 == 0 && stride_bg % 8 == 0 && stride_cm % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(c) & 7) == 0 && panels_fit(k, stride_am, stride_bk, stride_cm);
  if (swiglu && !vec)
    return fail(MOEGEMM_ERR_INVALID, "the SwiGLU epilogue needs the vector layout (LDS-DMA kernel)");
  rc = set_queue(p, queue);
  if (rc != MOEGEMM_OK) return rc;
  return launch(e, p, grid, vec, b_stream, stream);
}

int moegemm_grouped_mm_offs(const void* a, const void* b, void* c, const int32_t* offs, int32_t group_count,
                            int32_t rows, int32_t n, int32_t k, int64_t stride_am, int64_t stride_bg,
                            int64_t stride_bk, int64_t stride_cm, int32_t dtype, int32_t input_precision,
                            int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                            int32_t num_warps, int32_t num_stages, int32_t grid_size, int32_t b_stream, void* stream) {
  return offsets_impl(a, b, c, offs, group_count, rows, n, k, stride_am, stride_bg, stride_bk, stride_cm, dtype,
                      input_precision, block_m, block_n, block_k, group_size_m, num_warps, num_stages, grid_size,
                      false, nullptr, b_stream, stream);
}

int moegemm_grouped_mm_offs_swiglu(const void* a, const void* b, void* h, const int32_t* offs, int32_t group_count,
                                   int32_t rows, int32_t n, int32_t k, int64_t stride_am, int64_t stride_bg,
                                   int64_t stride_bk, int64_t stride_hm, int32_t dtype, int32_t block_m,
                                   int32_t block_n, int32_t block_k, int32_t group_size_m, int32_t num_warps,
                                   int32_t num_stages, int32_t grid_size, int32_t b_stream, void* stream) {
  return offsets_impl(a, b, h, offs, group_count, rows, n, k, stride_am, stride_bg, stride_bk, stride_hm, dtype,
                      MOEGEMM_PRECISION_IEEE, block_m, block_n, block_k, group_size_m, num_warps, num_stages,
                      grid_size, true, nullptr, b_stream, stream);
}

int moegemm_grouped_mm_offs_stealing(const void* a, const void* b, void* c, const int32_t* offs,
                                     int32_t group_count, int32_t rows, int32_t n, int32_t k, int64_t stride_am,
                                     int64_t stride_bg, int64_t stride_bk, int64_t stride_cm, int32_t dtype,
                                     int32_t input_precision, int32_t block_m, int32_t block_n, int32_t block_k,
                                     int32_t group_size_m, int32_t num_warps, int32_t num_stages,
                                     int32_t grid_size, void* queue, int32_t b_stream, void* stream) {
  if (!queue) return fail(MOEGEMM_ERR_INVALID, "the work-stealing launch needs a tile queue");
  return offsets_impl(a, b, c, offs, group_count, rows, n, k, stride_am, stride_bg, stride_bk, stride_cm, dtype,
                      input_precision, block_m, block_n, block_k, group_size_m, num_warps, num_stages, grid_size,
                      false, queue, b_stream, stream);
}

int moegemm_matmul(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k, int64_t stride_am,
                   int64_t stride_ak, int64_t stride_bk, int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
                   int32_t dtype, int32_t input_precision, int32_t block_m, int32_t block_n, int32_t block_k,
                   int32_t group_size_m, int32_t num_warps, int32_t num_stages, int32_t grid_size,
                   int32_t b_stream, void* stream) {
  const KernelEntry* e = nullptr;
  int rc = check_common(dtype, input_precision, group_size_m, &e, block_m, block_n, block_k, num_warps, num_stages);
  if (rc != MOEGEMM_OK) return rc;
  if (!a || !b || !c) return fail(MOEGEMM_ERR_INVALID, "matrix pointers must be non-null");
  if (m <= 0 || n <= 0 || k <= 0) return fail(MOEGEMM_ERR_INVALID, "shape must be positive (m=%d n=%d k=%d)", m, n, k);
  int64_t tiles = cdiv(m, block_m) * cdiv(n, block_n);
  if (tiles > INT32_MAX) return fail(MOEGEMM_ERR_INVALID, "tile count %lld exceeds int32", (long long)tiles);
  KParams p;
  std::memset(&p, 0, sizeof(p));
  p.mode = MODE_SINGLE;
  p.a = a;
  p.b = b;
  p.c = c;
  p.M = m;
  p.N = n;
  p.K = k;
  p.sam = stride_am;
  p.sak = stride_ak;
  p.sbk = stride_bk;
  p.sbn = stride_bn;
  p.scm = stride_cm;
  p.scn = stride_cn;
  p.G = 1;
  p.group_m = group_size_m;
  p.tf32 = input_precision == MOEGEMM_PRECISION_TF32;
  p.total_tiles = (int32_t)tiles;
  int grid = grid_size <= 0 ? p.total_tiles : (grid_size < p.total_tiles ? grid_size : p.total_tiles);
  return launch(e, p, grid, vector_layout_ok(a, b, c, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm,
                                           stride_cn, dtype), b_stream, stream);
}

}  // extern "C"
