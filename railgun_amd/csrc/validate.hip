// Opt-in checks of the indices the attention kernels trust.  Railgun's launchers pass block
// tables, context lengths and slot mappings to the kernels unchecked (an `unsafe` contract,
// crates/vllm-cuda/src/kernels/mod.rs:196-508), and so do the entries of this library: a bad
// block number or slot reads or writes outside the KV pool.  These entries scan the indices on
// the device and report the first bad one by name; they synchronise the stream, so they are a
// debugging aid, not for use inside a graph capture.
#include <mutex>
#include <vector>

#include "rg_common.hpp"

namespace rg {
namespace {

constexpr unsigned long long kNoError = 0x7F7F7F7F7F7F7F7FULL;  // the result cell before a scan

// One workgroup per sequence: code s * (max_blocks + 1) for a context length outside
// [0, max_blocks * block_size], s * (max_blocks + 1) + 1 + i for table entry i (one of the
// entries the context uses) outside [0, num_blocks).  The smallest code wins.
__global__ __launch_bounds__(256) void check_tables_kernel(const int32_t* __restrict__ bt,
                                                           const int32_t* __restrict__ ctx, int32_t max_blocks,
                                                           int32_t block_size, int32_t num_blocks,
                                                           unsigned long long* first_bad) {
  const int s = blockIdx.x;
  const int c = ctx[s];
  const unsigned long long base = (unsigned long long)s * (unsigned long long)(max_blocks + 1);
  if (c < 0 || (int64_t)c > (int64_t)max_blocks * block_size) {
    if (threadIdx.x == 0) atomicMin(first_bad, base);
    return;
  }
  const int used = (c + block_size - 1) / block_size;
  for (int i = threadIdx.x; i < used; i += blockDim.x) {
    const int32_t v = bt[(int64_t)s * max_blocks + i];
    if (v < 0 || v >= num_blocks) atomicMin(first_bad, base + 1 + (unsigned long long)i);
  }
}

// Slots at or past num_slots (negative slots are padding tokens, which the cache writes skip).
__global__ __launch_bounds__(256) void check_slots_kernel(const int32_t* __restrict__ slots, int32_t n,
                                                          int64_t num_slots, unsigned long long* first_bad) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if ((int64_t)slots[i] >= num_slots) atomicMin(first_bad, (unsigned long long)i);
  }
}

// Sets the result cell to kNoError (a kernel rather than a memset, so the stream carries
// kernels only).
__global__ void fill_cell_kernel(unsigned long long* cell) { *cell = kNoError; }

// The result cell of each device (allocated on first use, held until the process ends).
std::mutex g_cell_mutex;
std::vector<unsigned long long*> g_cells;

int result_cell(const char* op, unsigned long long** cell) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(RG_ERR_HIP, "%s: no current device", op);
  if ((int)g_cells.size() <= dev) g_cells.resize(dev + 1, nullptr);
  if (!g_cells[dev] && hipMalloc(reinterpret_cast<void**>(&g_cells[dev]), sizeof(unsigned long long)) != hipSuccess) {
    g_cells[dev] = nullptr;
    return fail(RG_ERR_HIP, "%s: cannot allocate the result cell", op);
  }
  *cell = g_cells[dev];
  return RG_OK;
}

// Fills the cell, runs `launch`, and returns the smallest code found (kNoError if none).
template <typename F>
int run_check(const char* op, hipStream_t s, F&& launch, unsigned long long* found) {
  unsigned long long* cell = nullptr;
  if (int st = result_cell(op, &cell)) return st;
  hipLaunchKernelGGL(fill_cell_kernel, dim3(1), dim3(1), 0, s, cell);
  if (int st = check_launch(op)) return st;
  launch(cell);
  if (int st = check_launch(op)) return st;
  if (hipMemcpyAsync(found, cell, sizeof(*found), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    return fail(RG_ERR_HIP, "%s: %s", op, hipGetErrorString(hipGetLastError()));
  }
  return RG_OK;
}

}  // namespace
}  // namespace rg

using namespace rg;

extern "C" int rg_validate_block_tables(const int32_t* block_table, const int32_t* context_lens, int32_t batch_size,
                                        int32_t max_blocks_per_seq, int32_t block_size, int32_t num_blocks,
                                        void* stream) {
  const char* op = "validate_block_tables";
  if (batch_size < 0 || max_blocks_per_seq < 0 || block_size <= 0 || num_blocks < 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: negative size or non-positive block_size", op);
  }
  if (batch_size == 0) return ok();
  if (!block_table || !context_lens) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  std::lock_guard<std::mutex> lock(g_cell_mutex);
  hipStream_t s = as_stream(stream);
  unsigned long long code = kNoError;
  int st = run_check(op, s, [&](unsigned long long* cell) {
    hipLaunchKernelGGL(check_tables_kernel, dim3(batch_size), dim3(256), 0, s, block_table, context_lens,
                       max_blocks_per_seq, block_size, num_blocks, cell);
  }, &code);
  if (st) return st;
  if (code == kNoError) return ok();
  const int64_t seq = (int64_t)(code / (unsigned long long)(max_blocks_per_seq + 1));
  const int64_t idx = (int64_t)(code % (unsigned long long)(max_blocks_per_seq + 1)) - 1;
  int32_t v = 0;
  const int32_t* src = idx < 0 ? context_lens + seq : block_table + seq * max_blocks_per_seq + idx;
  if (hipMemcpy(&v, src, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) {
    return fail(RG_ERR_HIP, "%s: reading the bad entry failed", op);
  }
  if (idx < 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: context_lens[%lld] = %d outside [0, %lld] (max_blocks_per_seq x block_size)",
                op, (long long)seq, v, (long long)max_blocks_per_seq * block_size);
  }
  return fail(RG_ERR_INVALID_ARGUMENT, "%s: block_table[%lld][%lld] = %d outside [0, %d) (the pool's blocks)", op,
              (long long)seq, (long long)idx, v, num_blocks);
}

extern "C" int rg_validate_slot_mapping(const int32_t* slot_mapping, int32_t num_tokens, int64_t num_slots,
                                        void* stream) {
  const char* op = "validate_slot_mapping";
  if (num_tokens < 0 || num_slots < 0) return fail(RG_ERR_INVALID_ARGUMENT, "%s: negative size", op);
  if (num_tokens == 0) return ok();
  if (!slot_mapping) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  std::lock_guard<std::mutex> lock(g_cell_mutex);
  hipStream_t s = as_stream(stream);
  unsigned long long code = kNoError;
  const unsigned grid = (unsigned)std::min<int64_t>(1024, ceil_div(num_tokens, 256));
  int st = run_check(op, s, [&](unsigned long long* cell) {
    hipLaunchKernelGGL(check_slots_kernel, dim3(grid), dim3(256), 0, s, slot_mapping, num_tokens, num_slots, cell);
  }, &code);
  if (st) return st;
  if (code == kNoError) return ok();
  int32_t v = 0;
  if (hipMemcpy(&v, slot_mapping + code, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) {
    return fail(RG_ERR_HIP, "%s: reading the bad entry failed", op);
  }
  return fail(RG_ERR_INVALID_ARGUMENT, "%s: slot_mapping[%llu] = %d not below %lld (the pool's slots; negative slots are "
              "padding)", op, code, v, (long long)num_slots);
}
