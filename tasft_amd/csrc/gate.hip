// Fused AttnGate forward for gfx950.
//
// Reference (tasft/modules/attn_gate.py:151-277):
//   qbar = mean over each block of bs tokens of Q (zero padded: the mean divides by bs)
//   kbar = same for K
//   logit[i, j] = w_out . relu(W_in . cat(qbar_i, kbar_j) + b_in)
//   soft = sigmoid(logit); if causal: soft[j > i] = 0 exactly; hard = soft >= tau
// The reference materialises cat(qbar_i, kbar_j) for every pair ([B,H,NB,NB,2D]).
// Since W_in . cat(x, y) = W_q x + W_k y with W_q = W_in[:, :D] and W_k = W_in[:, D:],
// this computes u_i = W_q qbar_i + b_in once per query block and v_j = W_k kbar_j once
// per key block, so each pair costs hidden x (add, max, fma) instead of a 2D-wide GEMV.
//
// Kernel 1 (pool + project) streams Q and K from HBM exactly once (GQA-native: K is
// pooled per KV head, never expanded). Kernel 2 (pairwise) evaluates the MLP for the
// causal pairs in fp32, applies sigmoid, the causal zero and the per-head threshold, and
// writes soft scores (fp32), optional logits, the uint8 hard mask and the active count.
// Flag bit 1 forces the diagonal blocks on in the hard mask (soft scores unchanged).
#include "common.h"

namespace tasft {

constexpr int kPoolBlocks = 8;    // blocks pooled per workgroup (amortises the W_in read)
constexpr int kGateMaxD = 256;
constexpr int kPairRows = 32;     // query-block rows per pairwise workgroup
constexpr int kPairCols = 64;     // key-block columns per inner tile
constexpr int kPairHid = 64;      // hidden units staged per LDS round

struct GatePoolParams {
  const uint16_t* q;
  const uint16_t* k;
  const float* w_in;  // [hidden, 2D]
  const float* b_in;  // [hidden]
  float* uq;          // [B, Hq, NB, hidden]
  float* uk;          // [B, Hkv, NB, hidden]
  unsigned long long* counter;
  int64_t sq[3], sk[3];
  int B, Hq, Hkv, S, D, bs, NB, hidden, chunks;
};

__global__ void __launch_bounds__(256)
gate_pool_project_kernel(const GatePoolParams p) {
  __shared__ float partial[256][8];  // per-thread 8-wide partial sums (row-group major)
  __shared__ float pooled[kPoolBlocks][kGateMaxD];

  const int tid = threadIdx.x;
  if (blockIdx.x == 0 && tid == 0 && p.counter) *p.counter = 0ull;

  const int64_t nq = (int64_t)p.B * p.Hq * p.chunks;
  const bool is_q = blockIdx.x < nq;
  const int64_t local = is_q ? blockIdx.x : blockIdx.x - nq;
  const int heads = is_q ? p.Hq : p.Hkv;
  const int64_t bh = local / p.chunks;
  const int chunk = (int)(local % p.chunks);
  const int b = (int)(bh / heads);
  const int h = (int)(bh % heads);
  const uint16_t* src = is_q ? p.q + b * p.sq[0] + h * p.sq[1] : p.k + b * p.sk[0] + h * p.sk[1];
  const int64_t srow = is_q ? p.sq[2] : p.sk[2];

  const int DOCT = p.D / 8;
  const int RG = 256 / DOCT;  // row groups
  const int dc = tid % DOCT;
  const int rg = tid / DOCT;
  const int blk0 = chunk * kPoolBlocks;
  const int nblk = min(kPoolBlocks, p.NB - blk0);
  const float inv_bs = 1.f / (float)p.bs;

  for (int bi = 0; bi < nblk; ++bi) {
    const int64_t t0 = (int64_t)(blk0 + bi) * p.bs;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (rg < RG) {
      for (int r = rg; r < p.bs; r += RG) {
        const int64_t tok = t0 + r;
        if (tok >= p.S) break;
        const u32x4_t v = *(const u32x4_t*)(src + tok * srow + dc * 8);
        float f[8];
        unpack_bf16x8(v, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += f[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) partial[tid][j] = acc[j];
    __syncthreads();
    for (int d = tid; d < p.D; d += 256) {
      const int c = d / 8, j = d % 8;
      float sum = 0.f;
      for (int g = 0; g < RG; ++g) sum += partial[g * DOCT + c][j];
      pooled[bi][d] = sum * inv_bs;
    }
    __syncthreads();
  }

  // Project: u[blk][c] = sum_d pooled[blk][d] * W_in[c][off + d] (+ b_in[c] for queries).
  const int off = is_q ? 0 : p.D;
  float* dst = (is_q ? p.uq : p.uk) + (bh * p.NB + blk0) * (int64_t)p.hidden;
  for (int i = tid; i < nblk * p.hidden; i += 256) {
    const int bi = i / p.hidden, c = i % p.hidden;
    const float* w = p.w_in + (int64_t)c * 2 * p.D + off;
    float acc = is_q ? p.b_in[c] : 0.f;
    for (int d = 0; d < p.D; d += 4) {
      const f32x4_t wv = *(const f32x4_t*)(w + d);
      acc = fmaf(pooled[bi][d + 0], wv[0], acc);
      acc = fmaf(pooled[bi][d + 1], wv[1], acc);
      acc = fmaf(pooled[bi][d + 2], wv[2], acc);
      acc = fmaf(pooled[bi][d + 3], wv[3], acc);
    }
    dst[(int64_t)bi * p.hidden + c] = acc;
  }
}

struct GatePairParams {
  const float* uq;
  const float* uk;
  const float* w_out;  // [hidden]
  const float* tau;    // [Hq]
  float* soft;         // [B, Hq, NB, NB]
  float* logits;       // [B, Hq, NB, NB] or null
  uint8_t* mask;       // [B, Hq, NB, NB]
  unsigned long long* counter;
  int B, Hq, Hkv, G, NB, hidden, causal, force_diag, row_tiles;
};

__global__ void __launch_bounds__(256)
gate_pairwise_kernel(const GatePairParams p) {
  __shared__ __attribute__((aligned(16))) float uq_t[kPairHid][kPairRows + 1];
  __shared__ __attribute__((aligned(16))) float uk_t[kPairHid][kPairCols + 4];
  __shared__ float wo[kPairHid];

  const int tid = threadIdx.x;
  const int tr = tid / 16;  // rows 2*tr, 2*tr+1
  const int tc = tid % 16;  // cols 4*tc .. 4*tc+3
  const int64_t bh = blockIdx.x / p.row_tiles;
  const int i0 = (int)(blockIdx.x % p.row_tiles) * kPairRows;
  const int b = (int)(bh / p.Hq);
  const int h = (int)(bh % p.Hq);
  const int kvh = h / p.G;
  const float tau = p.tau[h];
  const float* uq = p.uq + (bh * p.NB) * (int64_t)p.hidden;
  const float* uk = p.uk + (((int64_t)b * p.Hkv + kvh) * p.NB) * (int64_t)p.hidden;
  const int64_t obase = bh * (int64_t)p.NB * p.NB;
  const int i_last = min(i0 + kPairRows, p.NB) - 1;
  // With causal=1 and no logits requested, pairs above the diagonal are never evaluated.
  const bool skip_upper = p.causal && p.logits == nullptr;

  unsigned int active = 0;
  for (int j0 = 0; j0 < p.NB; j0 += kPairCols) {
    float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const bool compute = !(skip_upper && j0 > i_last);
    if (compute) {
      for (int c0 = 0; c0 < p.hidden; c0 += kPairHid) {
        const int hc = min(kPairHid, p.hidden - c0);
        __syncthreads();
        for (int e = tid; e < kPairRows * kPairHid; e += 256) {
          const int r = e / kPairHid, cc = e % kPairHid;
          const int i = i0 + r;
          uq_t[cc][r] = (cc < hc && i < p.NB) ? uq[(int64_t)i * p.hidden + c0 + cc] : 0.f;
        }
        for (int e = tid; e < kPairCols * kPairHid; e += 256) {
          const int r = e / kPairHid, cc = e % kPairHid;
          const int j = j0 + r;
          uk_t[cc][r] = (cc < hc && j < p.NB) ? uk[(int64_t)j * p.hidden + c0 + cc] : 0.f;
        }
        if (tid < kPairHid) wo[tid] = tid < hc ? p.w_out[c0 + tid] : 0.f;
        __syncthreads();
        for (int cc = 0; cc < hc; ++cc) {
          const float a0 = uq_t[cc][2 * tr];
          const float a1 = uq_t[cc][2 * tr + 1];
          const f32x4_t bv = *(const f32x4_t*)&uk_t[cc][4 * tc];
          const float w = wo[cc];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            acc[0][c] = fmaf(w, fmaxf(a0 + bv[c], 0.f), acc[0][c]);
            acc[1][c] = fmaf(w, fmaxf(a1 + bv[c], 0.f), acc[1][c]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int i = i0 + 2 * tr + r;
      if (i >= p.NB) continue;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = j0 + 4 * tc + c;
        if (j >= p.NB) continue;
        const float logit = acc[r][c];
        float soft = 1.f / (1.f + expf(-logit));
        if (p.causal && j > i) soft = 0.f;
        const bool on = soft >= tau || (p.force_diag && i == j);
        active += on ? 1u : 0u;
        const int64_t o = obase + (int64_t)i * p.NB + j;
        p.soft[o] = soft;
        p.mask[o] = on ? 1 : 0;
        if (p.logits) p.logits[o] = logit;
      }
    }
  }
  // One atomic per wave.
  const float tot = wave_sum((float)active);
  if ((tid & 63) == 0 && tot > 0.f) atomicAdd(p.counter, (unsigned long long)(tot + 0.5f));
}

}  // namespace tasft

using namespace tasft;

extern "C" size_t tasft_gate_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                             int64_t num_kv_heads, int64_t seq_len,
                                             int64_t block_size, int64_t hidden) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || block_size <= 0 ||
      hidden <= 0)
    return 0;
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  return (size_t)(batch * (num_q_heads + num_kv_heads) * nb * hidden) * sizeof(float) + 256;
}

extern "C" int tasft_gate_fwd(const void* q, const void* k, const float* w_in, const float* b_in,
                              const float* w_out, const float* thresholds, float* soft_scores,
                              float* logits, uint8_t* hard_mask, unsigned long long* active_count,
                              void* workspace, size_t workspace_bytes, int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                              int64_t head_dim, int64_t block_size, int64_t hidden,
                              const int64_t* q_strides, const int64_t* k_strides, int flags,
                              void* stream) {
  if (!q || !k || !w_in || !b_in || !w_out || !thresholds || !soft_scores || !hard_mask ||
      !active_count || !workspace || !q_strides || !k_strides)
    return set_error(kErrInvalidArgument, "gate: null pointer argument");
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || block_size <= 0 ||
      hidden <= 0)
    return set_error(kErrInvalidArgument, "gate: sizes must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "gate: num_q_heads must be a multiple of num_kv_heads");
  if (head_dim % 8 != 0 || head_dim > kGateMaxD || head_dim <= 0)
    return set_error(kErrUnsupported, "gate: head_dim must be a multiple of 8 and at most %d, got %lld",
                     kGateMaxD, (long long)head_dim);
  if (q_strides[3] != 1 || k_strides[3] != 1)
    return set_error(kErrInvalidArgument, "gate: head_dim must be the contiguous dimension");
  for (int j = 0; j < 3; ++j)
    if (q_strides[j] % 8 != 0 || k_strides[j] % 8 != 0)
      return set_error(kErrInvalidArgument, "gate: strides must be multiples of 8 elements");
  if ((((uintptr_t)q) & 15u) || (((uintptr_t)k) & 15u) || (((uintptr_t)w_in) & 15u))
    return set_error(kErrInvalidArgument, "gate: q, k and w_in must be 16-byte aligned");
  const size_t need = tasft_gate_workspace_bytes(batch, num_q_heads, num_kv_heads, seq_len,
                                                 block_size, hidden);
  if (workspace_bytes < need)
    return set_error(kErrWorkspace, "gate: workspace too small: need %zu bytes, got %zu", need,
                     workspace_bytes);
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  const int64_t chunks = (nb + kPoolBlocks - 1) / kPoolBlocks;
  const int64_t row_tiles = (nb + kPairRows - 1) / kPairRows;
  if (batch * (num_q_heads + num_kv_heads) * chunks > 0x7fffffffLL ||
      batch * num_q_heads * row_tiles > 0x7fffffffLL || seq_len > 0x3fffffffLL)
    return set_error(kErrUnsupported, "gate: problem too large for one launch");

  GatePoolParams pp;
  pp.q = (const uint16_t*)q;
  pp.k = (const uint16_t*)k;
  pp.w_in = w_in;
  pp.b_in = b_in;
  pp.uq = (float*)workspace;
  pp.uk = pp.uq + batch * num_q_heads * nb * hidden;
  pp.counter = active_count;
  for (int j = 0; j < 3; ++j) {
    pp.sq[j] = q_strides[j];
    pp.sk[j] = k_strides[j];
  }
  pp.B = (int)batch;
  pp.Hq = (int)num_q_heads;
  pp.Hkv = (int)num_kv_heads;
  pp.S = (int)seq_len;
  pp.D = (int)head_dim;
  pp.bs = (int)block_size;
  pp.NB = (int)nb;
  pp.hidden = (int)hidden;
  pp.chunks = (int)chunks;

  hipStream_t s = (hipStream_t)stream;
  const int64_t grid1 = batch * (num_q_heads + num_kv_heads) * chunks;
  hipLaunchKernelGGL(gate_pool_project_kernel, dim3((unsigned)grid1), dim3(256), 0, s, pp);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate: pool launch failed: %s", hipGetErrorString(err));

  GatePairParams qp;
  qp.uq = pp.uq;
  qp.uk = pp.uk;
  qp.w_out = w_out;
  qp.tau = thresholds;
  qp.soft = soft_scores;
  qp.logits = logits;
  qp.mask = hard_mask;
  qp.counter = active_count;
  qp.B = pp.B;
  qp.Hq = pp.Hq;
  qp.Hkv = pp.Hkv;
  qp.G = (int)(num_q_heads / num_kv_heads);
  qp.NB = pp.NB;
  qp.hidden = pp.hidden;
  qp.causal = (flags & 1) ? 1 : 0;
  qp.force_diag = (flags & 2) ? 1 : 0;
  qp.row_tiles = (int)row_tiles;
  const int64_t grid2 = batch * num_q_heads * row_tiles;
  hipLaunchKernelGGL(gate_pairwise_kernel, dim3((unsigned)grid2), dim3(256), 0, s, qp);
  if ((err = hipGetLastError()) != hipSuccess)
    return set_error(kErrLaunch, "gate: pairwise launch failed: %s", hipGetErrorString(err));
  return kOk;
}
