// Block-mask format conversion on gfx950.
//
// The reference passes block masks as dense boolean tensors [B, H, NBq, NBk]
// (tasft/kernels/block_sparse_fa.py:439-452) and its Triton kernel scans every byte of a
// row (:192-203). Callers that keep a selection as lists of block indices (a serving
// engine picking the top-k KV blocks per head) or that want the active blocks as
// compressed rows use these two conversions:
//
//   tasft_mask_compact:      dense block mask -> CSR (row_ptr, col_idx ascending), with an
//                            optional causal lower-triangle restriction (the AND the
//                            reference applies at :502-508);
//   tasft_mask_from_indices: padded index lists [rows, K] (-1 = empty slot) -> dense
//                            byte mask, the form the attention kernels read.
//
// Compaction is three launches: per-row counts (one wave per row, a ballot per 64
// columns), an exclusive scan of the counts in one workgroup, and the fill, in which
// each wave writes its row's column indices in ascending order from the same ballots.
#include "common.h"

#include "../../include/tasft_amd.h"

namespace tasft {

struct MaskView {
  const uint8_t* mask;
  int64_t s[4];  // byte strides of (b, h, row, col)
  int H, NBq, NBk;
  int causal;
};

__device__ __forceinline__ const uint8_t* mask_row(const MaskView& m, int64_t row) {
  const int64_t qb = row % m.NBq;
  const int64_t bh = row / m.NBq;
  const int64_t h = bh % m.H, b = bh / m.H;
  return m.mask + b * m.s[0] + h * m.s[1] + qb * m.s[2];
}

// Columns of row `row` that may be active: all, or the lower triangle incl. diagonal.
__device__ __forceinline__ int mask_row_end(const MaskView& m, int64_t row) {
  return m.causal ? min((int)(row % m.NBq) + 1, m.NBk) : m.NBk;
}

__global__ void __launch_bounds__(256) mask_count_kernel(const MaskView m, int64_t rows,
                                                         int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave; no barrier in this kernel
  const uint8_t* r = mask_row(m, row);
  const int end = mask_row_end(m, row);
  int cnt = 0;
  for (int c0 = 0; c0 < end; c0 += kWave) {
    const int c = c0 + lane;
    cnt += __popcll(__ballot(c < end && r[(int64_t)c * m.s[3]] != 0));
  }
  if (lane == 0) counts[row] = cnt;
}

// Exclusive scan of counts[0..rows) into row_ptr[0..rows], one workgroup of 1024
// threads walking the rows in tiles of 4096.
constexpr int kScanThreads = 1024;
constexpr int kScanPer = 4;

__global__ void __launch_bounds__(kScanThreads) mask_scan_kernel(const int32_t* counts, int64_t rows,
                                                                 int32_t* row_ptr) {
  __shared__ int wave_tot[kScanThreads / kWave];
  __shared__ int carry_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int carry = 0;
  for (int64_t t0 = 0; t0 < rows; t0 += (int64_t)kScanThreads * kScanPer) {
    int v[kScanPer];
    int sum = 0;
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) {
      const int64_t i = t0 + (int64_t)tid * kScanPer + e;
      v[e] = i < rows ? counts[i] : 0;
      sum += v[e];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += y;
    }
    if (lane == kWave - 1) wave_tot[wave] = incl;
    __syncthreads();
    int base = carry;
    for (int w = 0; w < wave; ++w) base += wave_tot[w];
    base += incl - sum;
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) {
      const int64_t i = t0 + (int64_t)tid * kScanPer + e;
      if (i < rows) row_ptr[i] = base;
      base += v[e];
    }
    if (tid == kScanThreads - 1) carry_lds = base;  // the last thread ends at the tile total
    __syncthreads();
    carry = carry_lds;
    __syncthreads();  // wave_tot and carry_lds are rewritten by the next tile
  }
  if (tid == 0) row_ptr[rows] = carry;
}

__global__ void __launch_bounds__(256) mask_fill_kernel(const MaskView m, int64_t rows,
                                                        const int32_t* row_ptr, int32_t* col_idx,
                                                        int64_t capacity) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave
  const uint8_t* r = mask_row(m, row);
  const int end = mask_row_end(m, row);
  int pos = row_ptr[row];
  for (int c0 = 0; c0 < end; c0 += kWave) {
    const int c = c0 + lane;
    const bool on = c < end && r[(int64_t)c * m.s[3]] != 0;
    const uint64_t bits = __ballot(on);
    const int64_t at = pos + __popcll(bits & ((1ull << lane) - 1ull));
    if (on && at < capacity) col_idx[at] = c;  // the caller sees overflow in row_ptr[rows]
    pos += __popcll(bits);
  }
}

// Index lists -> byte mask. One thread per (row, column) clears the mask; then one thread
// per list slot sets its column. Out-of-range indices (other than -1) raise the error
// flag and are skipped.
__global__ void __launch_bounds__(256) mask_clear_kernel(uint8_t* mask, int64_t rows, int ncols,
                                                         int* err) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i == 0) *err = 0;
  if (i < rows * ncols) mask[i] = 0;
}

__global__ void __launch_bounds__(256) mask_scatter_kernel(const int32_t* idx, int64_t rows, int k,
                                                           int64_t idx_row_stride, uint8_t* mask,
                                                           int ncols, int* err) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * k) return;
  const int64_t row = i / k, slot = i % k;
  const int c = idx[row * idx_row_stride + slot];
  if (c == -1) return;
  if (c < 0 || c >= ncols) {
    atomicOr(err, 1);
    return;
  }
  mask[row * ncols + c] = 1;
}

}  // namespace tasft

using namespace tasft;

extern "C" size_t tasft_mask_compact_workspace_bytes(int64_t batch, int64_t num_heads,
                                                     int64_t num_q_blocks) {
  if (batch <= 0 || num_heads <= 0 || num_q_blocks <= 0) return 0;
  return (size_t)(batch * num_heads * num_q_blocks) * sizeof(int32_t);
}

extern "C" int tasft_mask_compact(const uint8_t* block_mask, int64_t batch, int64_t num_heads,
                                  int64_t num_q_blocks, int64_t num_k_blocks,
                                  const int64_t* mask_strides, int causal, int32_t* row_ptr,
                                  int32_t* col_idx, int64_t col_capacity, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (!block_mask || !mask_strides || !row_ptr || !col_idx || !workspace)
    return set_error(kErrInvalidArgument, "mask_compact: null pointer argument");
  if (batch <= 0 || num_heads <= 0 || num_q_blocks <= 0 || num_k_blocks <= 0 || col_capacity < 0)
    return set_error(kErrInvalidArgument, "mask_compact: sizes must be positive");
  if (!strides_nonneg(mask_strides, 4))
    return set_error(kErrInvalidArgument, "mask_compact: strides must be non-negative");
  const int64_t rows = batch * num_heads * num_q_blocks;
  if (rows * num_k_blocks > 0x7fffffffLL || num_k_blocks > 0x7fffffffLL)
    return set_error(kErrUnsupported, "mask_compact: more than 2^31 mask entries");
  const size_t need = tasft_mask_compact_workspace_bytes(batch, num_heads, num_q_blocks);
  if (workspace_bytes < need)
    return set_error(kErrWorkspace, "mask_compact: workspace too small: need %zu bytes, got %zu",
                     need, workspace_bytes);
  MaskView m;
  m.mask = block_mask;
  for (int j = 0; j < 4; ++j) m.s[j] = mask_strides[j];
  m.H = (int)num_heads;
  m.NBq = (int)num_q_blocks;
  m.NBk = (int)num_k_blocks;
  m.causal = causal ? 1 : 0;
  int32_t* counts = (int32_t*)workspace;
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  hipLaunchKernelGGL(mask_count_kernel, dim3(grid), dim3(256), 0, s, m, rows, counts);
  hipLaunchKernelGGL(mask_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, counts, rows, row_ptr);
  hipLaunchKernelGGL(mask_fill_kernel, dim3(grid), dim3(256), 0, s, m, rows, row_ptr, col_idx,
                     col_capacity);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "mask_compact: launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" int tasft_mask_from_indices(const int32_t* indices, int64_t rows, int64_t k,
                                       int64_t index_row_stride, int64_t num_k_blocks,
                                       uint8_t* block_mask, int* error_flag, void* stream) {
  if (!indices || !block_mask || !error_flag)
    return set_error(kErrInvalidArgument, "mask_from_indices: null pointer argument");
  if (rows <= 0 || k < 0 || num_k_blocks <= 0 || index_row_stride < k)
    return set_error(kErrInvalidArgument, "mask_from_indices: invalid sizes");
  if (rows * num_k_blocks > 0x7fffffffLL || rows * (k > 0 ? k : 1) > 0x7fffffffLL)
    return set_error(kErrUnsupported, "mask_from_indices: more than 2^31 entries");
  hipStream_t s = (hipStream_t)stream;
  const int64_t n = rows * num_k_blocks;
  hipLaunchKernelGGL(mask_clear_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     block_mask, rows, (int)num_k_blocks, error_flag);
  if (k > 0) {
    const int64_t slots = rows * k;
    hipLaunchKernelGGL(mask_scatter_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, s,
                       indices, rows, (int)k, index_row_stride, block_mask, (int)num_k_blocks,
                       error_flag);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "mask_from_indices: launch failed: %s", hipGetErrorString(err));
  return kOk;
}
