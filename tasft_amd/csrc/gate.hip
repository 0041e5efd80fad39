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
// Pooling streams Q and K (bf16 or fp16, accumulated in fp32) from HBM exactly once
// (GQA-native: K is pooled per KV head, never expanded) in kernels that also project the
// block means. The pairwise stage evaluates the MLP for the causal pairs in fp32, applies
// sigmoid, the causal zero and the per-head threshold, and writes soft scores (fp32),
// optional logits, the uint8 hard mask and the active count. Flag bit 1 forces the
// diagonal blocks on in the hard mask (soft scores unchanged).
//
// Block size 64, D in {64, 128}, hidden a multiple of 32 up to 128 (the benchmarked gate):
// one kernel, gate_fused64_kernel, after a one-workgroup reset of its completion counters.
// Its first workgroups pool and project the key chunks; every other workgroup pools and
// projects one query chunk, waits for its KV group's key units and evaluates the chunk's
// rows. Otherwise one pooling launch (streaming for blocks 32, 64 and 128 with D in
// {64, 128}, generic else) is followed by gate_pairwise_kernel.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"

#include "../../include/tasft_amd.h"

namespace tasft {

constexpr int kPoolBlocks = 8;    // blocks pooled per workgroup (amortises the W_in read)
constexpr int kGateMaxD = 256;
constexpr int kPairHid = 64;      // hidden units staged per LDS round (pairwise)

struct GatePoolParams {
  const uint16_t* q;
  const uint16_t* k;
  const float* w_in;  // [hidden, 2D]
  const float* b_in;  // [hidden]
  float* uq;          // [B, Hq, NB, hidden]
  float* uk;          // [B, Hkv, NB, hidden]
  float* qmeans;      // [B, Hq, NB, D] block means of Q, or null
  float* kmeans;      // [B, Hkv, NB, D] block means of K, or null
  unsigned long long* counter;
  int64_t sq[3], sk[3];
  int64_t wg0;  // first workgroup index of the launch (gate_pool_proj64_kernel)
  int B, Hq, Hkv, S, D, bs, NB, hidden, chunks;
  int rotate;   // chunk-major query chunk order (query_chunk)
};

// Query chunk index g (0 .. B*Hq*chunks - 1) to its (b, head) and chunk: (b, head)-major,
// or with `rotate` chunk-major (g = chunk * B*Hq + bh), so that low indices are the early
// query rows (the cheapest under causal) and consecutive workgroups, which run on
// different XCDs, take different (b, head) of one chunk.
__device__ __forceinline__ void query_chunk(const GatePoolParams& p, int64_t g, int chunks,
                                            int64_t& bh, int& chunk) {
  if (p.rotate) {
    const int64_t nbh = (int64_t)p.B * p.Hq;
    bh = g % nbh;
    chunk = (int)(g / nbh);
  } else {
    bh = g / chunks;
    chunk = (int)(g % chunks);
  }
}

template <int DT>
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
        unpack16x8<DT>(v, f);
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
  float* mdst = is_q ? p.qmeans : p.kmeans;
  if (mdst) {
    mdst += (bh * p.NB + blk0) * (int64_t)p.D;
    for (int i = tid; i < nblk * p.D; i += 256) mdst[i] = pooled[i / p.D][i % p.D];
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


// Fast path for block size 64 and D in {64, 128}: one streaming kernel pools kFusePB
// blocks of one (batch, head) and projects their means. Each group of 4 blocks issues
// every row load up front through a buffer resource that ends at row S-1, so rows of a
// partial last block arrive as zeros, which is exactly the reference's zero padding (the
// mean still divides by the block size). The means stay in LDS; each thread then
// computes one hidden unit for 8 of the blocks from one read of its W_in row (the W_in
// halves are L2-resident), so the projection adds no HBM traffic and no launch.
constexpr int kFusePB = 16;
// Cache policy of the pooling loads: sc0 + nt (streamed: every byte of Q and K is read
// once here), measured 5% faster than the default policy.
constexpr int kStreamLoad = 3;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gate_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n, 0x00020000);
}

// Pools kFusePB blocks (chunk `chunk`) of BSZ rows (32, 64 or 128) of one (b, head) row stream
// of Q (is_q) or K and projects their means; `red` is the workgroup's LDS (4 x kFusePB x D
// floats).
template <int D, int DT, int BSZ = 64, bool PUBLISH = false>
__device__ __forceinline__ void pool_proj64(const GatePoolParams& p, bool is_q, int64_t bh,
                                            int chunk, float (&red)[4][kFusePB][D]) {
  static_assert(BSZ == 32 || BSZ == 64 || BSZ == 128, "block rows");
  constexpr int DOCT = D / 8;        // 16-byte chunks per row
  constexpr int RG = 256 / DOCT;     // row groups in the workgroup
  constexpr int RPT = BSZ / RG;      // rows per thread per block
  constexpr int WRG = kWave / DOCT;  // row groups per wave
  constexpr int GB = 256 / BSZ;      // blocks per load group (the same loads in flight)
  static_assert(WRG == 4 || WRG == 8, "row groups per wave");

  const int tid = threadIdx.x;
  const int heads = is_q ? p.Hq : p.Hkv;
  const int b = (int)(bh / heads);
  const int h = (int)(bh % heads);
  const uint16_t* src = is_q ? p.q + b * p.sq[0] + h * p.sq[1] : p.k + b * p.sk[0] + h * p.sk[1];
  const int srow = (int)(is_q ? p.sq[2] : p.sk[2]);
  const int blk0 = chunk * kFusePB;
  const int nblk = min(kFusePB, p.NB - blk0);
  const int row0 = blk0 * BSZ;
  const __amdgpu_buffer_rsrc_t r =
      gate_rsrc(src + (int64_t)row0 * srow, (int64_t)(p.S - row0) * srow * 2);

  const int dc = tid % DOCT, rg = tid / DOCT;
  const int wave = tid / kWave;
  for (int g = 0; g < nblk; g += GB) {
    u32x4_t v[GB][RPT];
#pragma unroll
    for (int bi = 0; bi < GB; ++bi)
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const int row = (g + bi) * BSZ + rg + RG * i;
        v[bi][i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                   r, (row * srow + dc * 8) * 2, 0, kStreamLoad));
      }
#pragma unroll
    for (int bi = 0; bi < GB; ++bi) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float f[8];
        unpack16x8<DT>(v[bi][i], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += f[j];
      }
      // Lanes l, l + DOCT, ... of a wave hold the same columns of different rows.
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = pair_sum32(acc[j]);
        x += __shfl_xor(x, 16, 64);
        if (WRG == 8) x += __shfl_xor(x, 8, 64);
        acc[j] = x;
      }
      if ((tid % kWave) < DOCT && g + bi < kFusePB) {
#pragma unroll
        for (int j = 0; j < 8; ++j) red[wave][g + bi][dc * 8 + j] = acc[j];
      }
    }
  }
  __syncthreads();
  // Block means, in place in red[0] (each element is read and written by one thread).
  const float inv_bs = 1.f / (float)BSZ;
  for (int e = tid; e < nblk * D; e += 256) {
    const int bi = e / D, d = e % D;
    red[0][bi][d] = ((red[0][bi][d] + red[1][bi][d]) + (red[2][bi][d] + red[3][bi][d])) * inv_bs;
  }
  __syncthreads();
  float* mdst = is_q ? p.qmeans : p.kmeans;
  if (mdst) {
    mdst += (bh * p.NB + blk0) * (int64_t)D;
    for (int e = tid; e < nblk * D; e += 256) mdst[e] = red[0][e / D][e % D];
  }

  // u[blk][c] = sum_d mean[blk][d] * W_in[c][off + d] (+ b_in[c] for query rows) on the
  // fp32 MFMA (v_mfma_f32_16x16x4_f32): M = the kFusePB = 16 blocks, N = 16 hidden units per
  // tile (tiles dealt to the four waves in turn), K = D. The reduction index is permuted so
  // that each lane reads contiguous runs: k-step s of lane group q = lane / 16 covers
  // d = q * D/4 + s (A and B use the same order). Lane l then holds A[l % 16][.] = the means
  // of block l % 16 and B[.][l % 16] = W_in row c0 + l % 16, and receives D[4q + r][l % 16]
  // for r = 0..3. The 16 W_in rows of a tile are first copied to a per-wave LDS area with
  // whole-line loads (two rows per instruction), since the operand order itself would touch
  // 64 cache lines per load.
  static_assert(kFusePB == 16, "one 16-row MFMA tile of blocks");
  constexpr int KQ = D / 4;      // k-steps per lane group
  constexpr int WCH = D / 4;     // 16-byte chunks per staged row
  static_assert(4 * 16 * D <= 4 * kFusePB * D, "W staging fits the pooling LDS");
  const int lane = tid % kWave, lr = lane % 16, lq = lane / 16;
  float a[KQ];
#pragma unroll
  for (int s4 = 0; s4 < KQ; s4 += 4) {
    const f32x4_t m4 = *(const f32x4_t*)&red[0][lr][lq * KQ + s4];
    a[s4] = m4[0], a[s4 + 1] = m4[1], a[s4 + 2] = m4[2], a[s4 + 3] = m4[3];
  }
  __syncthreads();  // every wave holds its means: the LDS is free for W staging
  // This wave's staging area: 16 rows x D floats, 16-byte chunk k of row r at position
  // k ^ (r & 7) (conflict-free operand reads).
  float* wst = &red[0][0][0] + wave * 16 * D;
  const int off = is_q ? 0 : D;
  float* dst = (is_q ? p.uq : p.uk) + (bh * p.NB + blk0) * (int64_t)p.hidden;
  const int ntiles = (p.hidden + 15) / 16;
  for (int nt = wave; nt < ntiles; nt += 4) {
    // Copy rows nt*16 .. +15 (rows past hidden read row 0; their results are not stored).
#pragma unroll
    for (int i = 0; i < (16 * WCH) / kWave; ++i) {
      const int e = i * kWave + lane, r = e / WCH, k = e % WCH;
      const int row = nt * 16 + r < p.hidden ? nt * 16 + r : 0;
      const f32x4_t v = *(const f32x4_t*)(p.w_in + (int64_t)row * 2 * D + off + 4 * k);
      *(f32x4_t*)(wst + r * D + 4 * (k ^ (r & 7))) = v;
    }
    const int c = nt * 16 + lr;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < KQ; s4 += 4) {
      const int k = (lq * KQ + s4) / 4;
      const f32x4_t w4 = *(const f32x4_t*)(wst + lr * D + 4 * (k ^ (lr & 7)));
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s4], w4[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s4 + 1], w4[1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s4 + 2], w4[2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s4 + 3], w4[3], acc, 0, 0, 0);
    }
    if (c < p.hidden) {
      const float bias = is_q ? p.b_in[c] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int blk = 4 * lq + r;
        if (blk >= nblk) continue;
        // PUBLISH: agent-scope atomic stores (written through to the device coherence
        // point), for units that workgroups on other XCDs read in the same launch.
        if (PUBLISH)
          __hip_atomic_store(dst + (int64_t)blk * p.hidden + c, acc[r] + bias, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        else
          dst[(int64_t)blk * p.hidden + c] = acc[r] + bias;
      }
    }
  }
}

// Workgroup wg0 + blockIdx.x pools query chunks first (B x Hq x chunks, see query_chunk),
// then key chunks.
template <int D, int DT, int BSZ = 64>
__global__ void __launch_bounds__(256)
gate_pool_proj64_kernel(const GatePoolParams p) {
  __shared__ __attribute__((aligned(16))) float red[4][kFusePB][D];  // per-wave sums, then means
  if (blockIdx.x == 0 && threadIdx.x == 0 && p.counter) *p.counter = 0ull;
  const int chunks = (p.NB + kFusePB - 1) / kFusePB;
  const int64_t nq = (int64_t)p.B * p.Hq * chunks;
  const int64_t wg = (int64_t)blockIdx.x + p.wg0;
  if (wg < nq) {
    int64_t bh;
    int chunk;
    query_chunk(p, wg, chunks, bh, chunk);
    pool_proj64<D, DT, BSZ>(p, true, bh, chunk, red);
  } else {
    pool_proj64<D, DT, BSZ>(p, false, (wg - nq) / chunks, (int)((wg - nq) % chunks), red);
  }
}

struct GatePairParams {
  const float* uq;
  const float* uk;
  const float* w_out;  // [hidden]
  const float* tau;    // [Hq]
  float* soft;         // [B, Hq, NBq, NBk]
  float* logits;       // [B, Hq, NBq, NBk] or null
  uint8_t* mask;       // [B, Hq, NBq, NBk]
  unsigned long long* counter;
  // uq holds NBq query-block rows whose global block index is row0 + i (a decode step:
  // one row); uk holds NBk key blocks. The causal zero and the forced diagonal compare
  // key block j with the global query block row0 + i.
  int B, Hq, Hkv, G, NBq, NBk, row0, hidden, causal, force_diag, tiles_q, tiles_k;
  int64_t uk_bh_stride;  // elements between the key units of consecutive (b, KV head)
};

// Pairwise MLP: a workgroup evaluates a kPairTile x kPairTile tile of (query block,
// key block) pairs of one (batch, head). With relu(x) = (x + |x|) / 2,
//   logit[i][j] = sum_c w_c relu(u_ic + v_jc)
//               = (A_i + B_j) / 2 + (sum_c w_c |u_ic + v_jc|) / 2,  A_i = sum_c w_c u_ic,
// so each (pair, unit) costs one add and one fma with an |.| source modifier instead of
// add, max and fma. The hidden units are staged kPairHid at a time (transposed) and
// split over the four waves, 32 each; lane (tr, tc) of a wave accumulates the 4 x 4 pairs
// rows 4tr.., cols 4tc.. (three LDS reads per 16 pairs and hidden unit). The four
// partial sums meet in LDS; the epilogue applies sigmoid, the causal zero and the
// threshold with coalesced stores.
constexpr int kPairTile = 32;
constexpr int kPairLd = kPairTile + 4;
// Row r of staged unit cc sits at position r ^ 4 * ((cc / 8) % 8) of its LDS row: the eight
// threads that stage one tile row write units eight apart, which the swizzle spreads over
// different banks; runs of four rows (r % 4 == 0) stay contiguous and 16-byte aligned.
__device__ __forceinline__ int pair_swz(int cc, int r) { return r ^ (4 * ((cc >> 3) & 7)); }

__global__ void __launch_bounds__(256)
gate_pairwise_kernel(const GatePairParams p) {
  // [kPairHid][kPairLd] query units | [kPairHid][kPairLd] key units; afterwards the four
  // partial-sum tiles [4][kPairTile][kPairLd] (the same size).
  __shared__ __attribute__((aligned(16))) float lds[2 * kPairHid * kPairLd];
  __shared__ float wo[kPairHid];
  __shared__ float ab[2][kPairTile];  // A_i of the tile's query rows, B_j of its key rows
  static_assert(2 * kPairHid >= 4 * kPairTile, "partial sums alias the staging tiles");
  __shared__ unsigned int wave_count[4];
  float* uq_t = lds;
  float* uk_t = lds + kPairHid * kPairLd;

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int tr = lane / 8, tc = lane % 8;
  const int per_head = p.tiles_q * p.tiles_k;
  const int64_t bh = blockIdx.x / per_head;
  const int t2 = (int)(blockIdx.x % per_head);
  const int i0 = (t2 / p.tiles_k) * kPairTile;
  const int j0 = (t2 % p.tiles_k) * kPairTile;
  const int b = (int)(bh / p.Hq);
  const int h = (int)(bh % p.Hq);
  const int kvh = h / p.G;
  const float* uq = p.uq + (bh * p.NBq) * (int64_t)p.hidden;
  const float* uk = p.uk + ((int64_t)b * p.Hkv + kvh) * p.uk_bh_stride;
  // With causal=1 and no logits requested, a tile wholly above the diagonal is never
  // evaluated (its soft scores are exactly zero).
  const bool skip = p.causal && p.logits == nullptr && j0 > p.row0 + i0 + kPairTile - 1;

  if (!skip) {
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[r][c] = 0.f;
    float a_part = 0.f, b_part = 0.f;             // this thread's share of A_sr and B_sr
    constexpr int SU = kPairHid / 8;              // units staged per thread
    const int sr = tid / 8, su = (tid % 8) * SU;  // staging: row sr, units su..su+SU-1
    const bool vec = (p.hidden % 4) == 0;         // rows start 16-byte aligned
    for (int c0 = 0; c0 < p.hidden; c0 += kPairHid) {
      const int hc = min(kPairHid, p.hidden - c0);
      if (c0 > 0) __syncthreads();
      const int i = i0 + sr, j = j0 + sr;
      const float* qrow = uq + (int64_t)i * p.hidden + c0;
      const float* krow = uk + (int64_t)j * p.hidden + c0;
      if (vec && su + SU <= hc) {
        // Whole run in range: 16-byte loads (hc is a multiple of 4 here).
#pragma unroll
        for (int u = 0; u < SU; u += 4) {
          const f32x4_t a = i < p.NBq ? *(const f32x4_t*)(qrow + su + u) : (f32x4_t){};
          const f32x4_t c = j < p.NBk ? *(const f32x4_t*)(krow + su + u) : (f32x4_t){};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float w = p.w_out[c0 + su + u + e];
            const int cc = su + u + e;
            uq_t[cc * kPairLd + pair_swz(cc, sr)] = a[e];
            uk_t[cc * kPairLd + pair_swz(cc, sr)] = c[e];
            a_part = fmaf(w, a[e], a_part);
            b_part = fmaf(w, c[e], b_part);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < SU; ++u) {
          const int cc = su + u;
          const float a = (cc < hc && i < p.NBq) ? qrow[cc] : 0.f;
          const float c = (cc < hc && j < p.NBk) ? krow[cc] : 0.f;
          const float w = cc < hc ? p.w_out[c0 + cc] : 0.f;
          uq_t[cc * kPairLd + pair_swz(cc, sr)] = a;
          uk_t[cc * kPairLd + pair_swz(cc, sr)] = c;
          a_part = fmaf(w, a, a_part);
          b_part = fmaf(w, c, b_part);
        }
      }
      if (tid < kPairHid) wo[tid] = tid < hc ? p.w_out[c0 + tid] : 0.f;
      __syncthreads();
      // Wave w takes units w, w+4, ...; units past hc (up to the next multiple of 4)
      // are zero in every operand and contribute nothing.
      const int nu = (hc + 3) / 4;
#pragma unroll 8
      for (int u = 0; u < nu; ++u) {
        const int cc = 4 * u + wave;
        const f32x4_t av = *(const f32x4_t*)&uq_t[cc * kPairLd + pair_swz(cc, 4 * tr)];
        const f32x4_t bv = *(const f32x4_t*)&uk_t[cc * kPairLd + pair_swz(cc, 4 * tc)];
        const float w = wo[cc];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[r][c] = fmaf(fabsf(av[r] + bv[c]), w, acc[r][c]);
      }
    }
    // The 8 threads that staged row sr are consecutive lanes.
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
      a_part += __shfl_xor(a_part, off, kWave);
      b_part += __shfl_xor(b_part, off, kWave);
    }
    if ((tid & 7) == 0) {
      ab[0][sr] = a_part;
      ab[1][sr] = b_part;
    }
    __syncthreads();
    float* part = lds + wave * (kPairTile * kPairLd);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *(f32x4_t*)&part[(4 * tr + r) * kPairLd + 4 * tc] =
          (f32x4_t){acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
    __syncthreads();
  }

  const float tau = p.tau[h];
  const int64_t obase = bh * (int64_t)p.NBq * p.NBk;
  unsigned int active = 0;
#pragma unroll
  for (int k = 0; k < (kPairTile * kPairTile) / 256; ++k) {
    const int idx = tid + 256 * k;
    const int ii = idx / kPairTile, jj = idx % kPairTile;
    const int i = i0 + ii, j = j0 + jj;
    if (i >= p.NBq || j >= p.NBk) continue;
    float logit = 0.f;
    if (!skip) {
      const int o = ii * kPairLd + jj;
      const int t = kPairTile * kPairLd;
      const float sabs = (lds[o] + lds[t + o]) + (lds[2 * t + o] + lds[3 * t + o]);
      logit = 0.5f * ((ab[0][ii] + ab[1][jj]) + sabs);
    }
    float soft = 1.f / (1.f + expf(-logit));
    if (p.causal && j > p.row0 + i) soft = 0.f;
    const bool on = soft >= tau || (p.force_diag && p.row0 + i == j);
    active += on ? 1u : 0u;
    const int64_t o = obase + (int64_t)i * p.NBk + j;
    p.soft[o] = soft;
    p.mask[o] = on ? 1 : 0;
    if (p.logits) p.logits[o] = logit;
  }
  // One atomic per workgroup: same-address atomics serialise in L2, so a per-wave
  // atomic costs more than the extra barrier.
  const float tot = wave_sum((float)active);
  if (lane == 0) wave_count[wave] = (unsigned int)(tot + 0.5f);
  __syncthreads();
  if (tid == 0) {
    const unsigned int t = (wave_count[0] + wave_count[1]) + (wave_count[2] + wave_count[3]);
    if (t) atomicAdd(p.counter, (unsigned long long)t);
  }
}

// Query pooling and the pairwise MLP in one kernel (block size 64, D in {64, 128}, hidden a
// multiple of kFuseHid and at most kFuseMaxHid). It runs after gate_pool_proj64_kernel has
// projected every key block (that launch covers the key chunks only), so a workgroup
// depends on no other workgroup of its own launch: it pools and projects query chunk
// `chunk` of one (b, head) (kFusePB query-block rows), then evaluates those rows against
// the key blocks they need (blocks 0 .. chunk end under causal without logits, all blocks
// otherwise) and writes the rows' soft scores, hard mask and logits.
//
// Pairwise layout: key blocks in groups of kFuseKeys = 128, 32 per wave. The chunk's query
// units (all hidden units) and w_out are staged once, transposed, for the workgroup; each
// wave stages the units of its own 32 key blocks, kFuseHid at a time, in its own LDS area,
// with the next round's loads in flight during the current round's MLP, so the rounds need
// no workgroup barrier. Lane (tr, tc) accumulates rows 2tr, 2tr+1 against keys 4tc ..
// 4tc+3 of its wave over every hidden unit. The logit uses the same relu(x) = (x + |x|) / 2
// split as gate_pairwise_kernel, with A_i and B_j summed in a fixed order.
constexpr int kFuseHid = 32;
constexpr int kFuseMaxHid = 128;
constexpr int kFuseKeys = 128;
constexpr int kFuseLdq = kFusePB + 4;
constexpr int kFuseLdw = 32 + 4;
constexpr int kFuseWave = kFuseHid * kFuseLdw + 32;  // one wave's key units + its B_j
constexpr int kFuseFloats = kFuseMaxHid * kFuseLdq + kFuseMaxHid + 16 * kFusePB + kFusePB +
                            4 * kFuseWave;

// The pairwise rows of query chunk `chunk` of (b, head) `bh`, whose units are in q.uq: the
// chunk's query units and w_out staged once, A_i, then the key blocks in groups of
// kFuseKeys (see the layout note above), sigmoid, causal zero, tau and the forced
// diagonal; the chunk's active count is added to q.counter. `keys_ready` is called by every
// thread before the first key unit is read and returns whether the key units may be read.
template <typename KeysReady>
__device__ __forceinline__ void pair_chunk64(const GatePairParams& q, int64_t bh, int chunk,
                                             float* lds, unsigned int* wave_count,
                                             KeysReady&& keys_ready) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int tr = lane / 8, tc = lane % 8;
  const int b = (int)(bh / q.Hq), h = (int)(bh % q.Hq), kvh = h / q.G;
  const int i0 = chunk * kFusePB;
  const int nrows = min(kFusePB, q.NBq - i0);
  const int hid = q.hidden;
  const float* uq = q.uq + (bh * q.NBq + i0) * (int64_t)hid;
  const float* uk = q.uk + ((int64_t)b * q.Hkv + kvh) * q.uk_bh_stride;
  const int kneed = (q.causal && q.logits == nullptr) ? min(i0 + kFusePB, q.NBk) : q.NBk;
  const float tau = q.tau[h];
  float* uq_t = lds;                            // [hid][kFuseLdq]
  float* wo = uq_t + kFuseMaxHid * kFuseLdq;    // [hid]
  float* apart = wo + kFuseMaxHid;              // [16][kFusePB] partial A_i
  float* arow = apart + 16 * kFusePB;           // A_i [kFusePB]
  float* wst = arow + kFusePB + wave * kFuseWave;  // this wave: [kFuseHid][kFuseLdw] units
  float* bkey = wst + kFuseHid * kFuseLdw;         // this wave: B_j of its 32 keys

  // The chunk's units were stored by all four waves, and the pooling LDS is reused below.
  __syncthreads();
  {
    const int row = tid % kFusePB;
    for (int u4 = tid / kFusePB; 4 * u4 < hid; u4 += 256 / kFusePB) {
      const f32x4_t v = row < nrows ? *(const f32x4_t*)(uq + (int64_t)row * hid + 4 * u4)
                                    : (f32x4_t){};
#pragma unroll
      for (int e = 0; e < 4; ++e) uq_t[(4 * u4 + e) * kFuseLdq + row] = v[e];
    }
    for (int c = tid; c < hid; c += 256) wo[c] = q.w_out[c];
  }
  __syncthreads();
  {
    // A_i: sixteen groups of hid / 16 units per row, then the groups in order.
    const int row = tid % kFusePB, g = tid / kFusePB, per = hid / 16;
    float a = 0.f;
    for (int c = g * per; c < (g + 1) * per; ++c) a = fmaf(wo[c], uq_t[c * kFuseLdq + row], a);
    apart[g * kFusePB + row] = a;
  }
  __syncthreads();
  if (tid < kFusePB) {
    float a = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) a += apart[g * kFusePB + tid];
    arow[tid] = a;
  }
  __syncthreads();

  // The key units are read from here on: the caller's wait for them (a no-op when an
  // earlier launch wrote them). Without them the chunk's rows get NaN scores and an empty
  // mask, and nothing is added to the active count.
  if (!keys_ready()) {
    for (int e = tid; e < nrows * q.NBk; e += 256) {
      const int64_t o = (bh * q.NBq + i0 + e / q.NBk) * (int64_t)q.NBk + e % q.NBk;
      // The quiet-NaN bit pattern, stored as an integer (the build assumes no NaN arithmetic).
      reinterpret_cast<uint32_t*>(q.soft)[o] = 0x7fc00000u;
      q.mask[o] = 0;
      if (q.logits) reinterpret_cast<uint32_t*>(q.logits)[o] = 0x7fc00000u;
    }
    return;
  }

  // Staging role of this lane: key block kk of the wave's 32, units 16*hh .. +15 of a round.
  const int kk = lane % 32, hh = lane / 32;
  const bool vec_out = (q.NBk % 4) == 0;
  unsigned int active = 0;
  for (int k0 = 0; k0 < q.NBk; k0 += kFuseKeys) {
    const int kw = k0 + 32 * wave;  // first key block of this wave
    const bool wave_on = kw < kneed;
    float acc[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][e] = 0.f;
    if (wave_on) {
      const int j = kw + kk;
      const bool kin = j < q.NBk;
      const float* ksrc = uk + (int64_t)j * hid + 16 * hh;
      f32x4_t kv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[i] = kin ? *(const f32x4_t*)(ksrc + 4 * i) : (f32x4_t){};
      float b_part = 0.f;
      for (int c0 = 0; c0 < hid; c0 += kFuseHid) {
        // LDS accesses of one wave execute in order: the previous round's reads of this
        // area are done before these writes, and these writes before the reads below. The
        // wave barriers keep the compiler from reordering them.
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int cc = 16 * hh + 4 * i + e;
            wst[cc * kFuseLdw + kk] = kv[i][e];
            b_part = fmaf(wo[c0 + cc], kv[i][e], b_part);
          }
        __builtin_amdgcn_wave_barrier();
        if (c0 + kFuseHid < hid) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            kv[i] = kin ? *(const f32x4_t*)(ksrc + c0 + kFuseHid + 4 * i) : (f32x4_t){};
        }
#pragma unroll 8
        for (int cc = 0; cc < kFuseHid; ++cc) {
          const f32x2_t av = *(const f32x2_t*)&uq_t[(c0 + cc) * kFuseLdq + 2 * tr];
          const f32x4_t bv = *(const f32x4_t*)&wst[cc * kFuseLdw + 4 * tc];
          const float w = wo[c0 + cc];
#pragma unroll
          for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[r][e] = fmaf(fabsf(av[r] + bv[e]), w, acc[r][e]);
        }
      }
      // B_j of key kk: its two unit halves, held by lanes kk and kk + 32.
      const float bj = b_part + __shfl_xor(b_part, 32, kWave);
      __builtin_amdgcn_wave_barrier();
      if (hh == 0) bkey[kk] = bj;
      __builtin_amdgcn_wave_barrier();
    }
    // Rows 2tr + r, keys kw + 4tc + e. Keys at or past kneed are above the diagonal of
    // every row here (causal, no logits): their soft scores are exactly 0.
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ii = 2 * tr + r, i = i0 + ii;
      if (ii >= nrows) continue;
      float soft[4], lg[4];
      uint32_t on4 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int jk = kw + 4 * tc + e;
        float logit = 0.f;
        if (wave_on) logit = 0.5f * ((arow[ii] + bkey[4 * tc + e]) + acc[r][e]);
        float sv = 1.f / (1.f + expf(-logit));
        if (q.causal && jk > q.row0 + i) sv = 0.f;
        const bool on = jk < q.NBk && (sv >= tau || (q.force_diag && q.row0 + i == jk));
        active += on ? 1u : 0u;
        on4 |= (on ? 1u : 0u) << (8 * e);
        soft[e] = sv;
        lg[e] = logit;
      }
      const int j0 = kw + 4 * tc;
      const int64_t o = (bh * q.NBq + i) * (int64_t)q.NBk + j0;
      if (vec_out && j0 + 4 <= q.NBk) {
        *(f32x4_t*)(q.soft + o) = (f32x4_t){soft[0], soft[1], soft[2], soft[3]};
        *(uint32_t*)(q.mask + o) = on4;
        if (q.logits) *(f32x4_t*)(q.logits + o) = (f32x4_t){lg[0], lg[1], lg[2], lg[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (j0 + e >= q.NBk) break;
          q.soft[o + e] = soft[e];
          q.mask[o + e] = (uint8_t)((on4 >> (8 * e)) & 1u);
          if (q.logits) q.logits[o + e] = lg[e];
        }
      }
    }
  }
  const float tot = wave_sum((float)active);
  if (lane == 0) wave_count[wave] = (unsigned int)(tot + 0.5f);
  __syncthreads();
  if (tid == 0) {
    const unsigned int t = (wave_count[0] + wave_count[1]) + (wave_count[2] + wave_count[3]);
    if (t) atomicAdd(q.counter, (unsigned long long)t);
  }
}


// ---------------------------------------------------------------------------------------
// One-launch gate (block 64, D 64 or 128, hidden a multiple of kFuseHid up to kFuseMaxHid).
//
// Workgroups 0 .. nk-1 pool and project the key chunks of every (b, KV head), then raise
// that group's completion counter. Each later workgroup pools and projects one query
// chunk, stages its units and A_i, waits until every key chunk of its group is complete,
// and evaluates its rows (pair_chunk64). Query chunks run in reverse chunk-major order:
// the late query rows (the longest MLP) start first, and the workgroups dispatched last,
// once key workgroups have left, take the early rows, whose MLP is short.
//
// Publication at agent scope without an L2 writeback: a key workgroup stores its units
// with agent-scope atomic stores (written through to the device coherence point), waits
// for them (vmcnt(0)), meets the workgroup barrier, and thread 0 adds 1 to the group's
// counter with a relaxed agent-scope atomic. Thread 0 of a query workgroup polls the
// counter with relaxed agent-scope loads (device-level reads) and s_sleep, then runs one
// agent-scope acquire fence (this CU's L1 and the XCD's L2 invalidated) before the barrier
// that releases every thread's unit reads. Measured on the box with a bounded probe: a
// counter raised on one XCD is seen by pollers on all eight, and the data published with it
// reads back exactly.
//
// The wait cannot deadlock: a workgroup waits only on workgroups of lower index, which wait
// on nothing, and each XCD dispatches its workgroups in index order. It is bounded anyway
// by the wall clock (s_memrealtime, 100 MHz): after kGateWaitTicks the workgroup gives up,
// writes NaN scores and an empty mask for its rows and sets bit 63 of the active count,
// which the host reports as an error.
// ---------------------------------------------------------------------------------------
constexpr unsigned long long kGateWaitTicks = 100000;  // 1 ms
constexpr int kGateSyncStride = 16;                   // u32 per completion counter (64 bytes)
constexpr unsigned long long kGateTimeoutBit = 1ull << 63;

struct GateSync {
  unsigned int* done;  // [B * Hkv] completion counters, kGateSyncStride apart, zeroed per call
  unsigned long long wait_ticks;  // bound of a query workgroup's wait (kGateWaitTicks)
  // Diagnostic (tasft_gate_debug_wait_fault): key workgroups do not raise their counter, so
  // every wait runs into its bound and the error path is taken.
  int skip_publish;
};

template <int D, int DT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
gate_fused64_kernel(const GatePoolParams p, const GatePairParams q, const GateSync sy) {
  constexpr int kRed = 4 * kFusePB * D;
  constexpr int kLds = kRed > kFuseFloats + 8 ? kRed : kFuseFloats + 8;
  // The pooling sums, then the pairwise staging; the per-wave counts and the wait result
  // sit past the staging area, so the workgroup needs exactly kLds floats (32 KB at D 128:
  // five workgroups per CU, every workgroup of config 2 resident at once).
  __shared__ __attribute__((aligned(16))) float lds[kLds];
  unsigned int* wave_count = reinterpret_cast<unsigned int*>(lds + kFuseFloats);
  int& ready_s = *reinterpret_cast<int*>(lds + kFuseFloats + 4);
  static_assert(kFuseHid == 32 && kFusePB == 16 && kFuseKeys == 128, "thread layouts");

  auto& red = *reinterpret_cast<float(*)[4][kFusePB][D]>(lds);
  const int fchunks = (p.NB + kFusePB - 1) / kFusePB;
  const int64_t nk = (int64_t)p.B * p.Hkv * fchunks;
  const int64_t nq = (int64_t)p.B * p.Hq * fchunks;
  const int64_t wg = blockIdx.x;
  if (wg < nk) {
    const int64_t bkv = wg / fchunks;
    pool_proj64<D, DT, 64, true>(p, false, bkv, (int)(wg % fchunks), red);
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this thread's unit stores are performed
    __syncthreads();
    if (threadIdx.x == 0 && !sy.skip_publish)
      __hip_atomic_fetch_add(sy.done + bkv * kGateSyncStride, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  int64_t bh;
  int chunk;
  query_chunk(p, nq - 1 - (wg - nk), fchunks, bh, chunk);
  pool_proj64<D, DT>(p, true, bh, chunk, red);
  const int b = (int)(bh / q.Hq), kvh = (int)(bh % q.Hq) / q.G;
  const unsigned int* cnt = sy.done + ((int64_t)b * q.Hkv + kvh) * kGateSyncStride;
  pair_chunk64(q, bh, chunk, lds, wave_count, [&]() -> bool {
    if (threadIdx.x == 0) {
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      int ok = 0;
      for (;;) {
        if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= (unsigned)fchunks) {
          ok = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > sy.wait_ticks) break;
        __builtin_amdgcn_s_sleep(8);
      }
      if (!ok) atomicOr(q.counter, kGateTimeoutBit);
      ready_s = ok;
      // One acquire for the workgroup: it invalidates this CU's L1 and the XCD's L2 lines,
      // which the barrier below orders before every thread's unit reads.
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    return ready_s != 0;
  });
}

// Zeroes the completion counters of gate_fused64_kernel and the active count (a kernel on
// the caller's stream, so the call can be captured in a graph).
__global__ void __launch_bounds__(256)
gate_sync_reset_kernel(unsigned int* done, int n, unsigned long long* counter) {
  for (int i = threadIdx.x; i < n; i += 256) done[(int64_t)i * kGateSyncStride] = 0u;
  if (threadIdx.x == 0) *counter = 0ull;
}

// One cached decode step's gate rows, for a KV head and its G <= kRowMaxG query heads per
// workgroup. It adds the new token's key and queries to the running sums of its block
// (reset first at a block start), projects the sums (W_in halves transposed with 1/block
// folded in, so a zero-padded block mean is sum x W), stores the key unit of the
// current block `row` among the kept units, and evaluates the rows of the G heads against
// key blocks 0 .. row: logit = w_out . relu(u + v_j), sigmoid, per-head tau, the forced
// diagonal. Thread j takes key block j (and j + 256, ...), all G heads at once.
constexpr int kRowMaxG = 8;
constexpr int kRowMaxHid = 256;

struct GateDecodeRowParams {
  const uint16_t* q_new;  // [B, Hq, D] (16-bit), strides sq
  const uint16_t* k_new;  // [B, Hkv, D], strides sk
  int64_t sq[2], sk[2];
  float* q_sum;           // [B, Hq, D]
  float* k_sum;           // [B, Hkv, D]
  float* uk;              // kept key units, block j of (b, KV head g) at (b*Hkv+g)*uk_stride + j*hidden
  int64_t uk_stride;
  const float* wq_t;      // [D, hidden]
  const float* wk_t;      // [D, hidden]
  const float* b_in;      // [hidden]
  const float* w_out;     // [hidden]
  const float* tau;       // [Hq]
  float* soft;            // [B, Hq, 1, row + 1]
  uint8_t* mask;          // [B, Hq, 1, row + 1]
  unsigned long long* counter;
  int B, Hq, Hkv, G, D, hidden, row, reset, force_diag;
};

// MG: the query heads per KV head rounded up to 1, 2, 4 or 8; heads G .. MG - 1 are zero and
// never stored, so the loops carry no per-head branch.
template <int DT, int MG>
__global__ void __launch_bounds__(256)
gate_decode_row_kernel(const GateDecodeRowParams p) {
  __shared__ float ks[kGateMaxD];
  __shared__ float qs[MG][kGateMaxD];
  __shared__ __attribute__((aligned(16))) float u[MG][kRowMaxHid];
  __shared__ __attribute__((aligned(16))) float vrow[kRowMaxHid];
  __shared__ float wo[kRowMaxHid];
  __shared__ unsigned int wave_count[4];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int b = blockIdx.x / p.Hkv, kvh = blockIdx.x % p.Hkv;
  const int h0 = kvh * p.G;
  const int D = p.D, hid = p.hidden;
  for (int d = tid; d < D; d += 256) {
    const float kn = bits16_to_f32<DT>(p.k_new[b * p.sk[0] + kvh * p.sk[1] + d]);
    float* ksp = p.k_sum + ((int64_t)b * p.Hkv + kvh) * D + d;
    const float v = (p.reset ? 0.f : *ksp) + kn;
    *ksp = v;
    ks[d] = v;
  }
  for (int e = tid; e < MG * D; e += 256) {
    const int g = e / D, d = e % D, h = h0 + g;
    if (g >= p.G) {
      qs[g][d] = 0.f;
      continue;
    }
    const float qn = bits16_to_f32<DT>(p.q_new[b * p.sq[0] + h * p.sq[1] + d]);
    float* qsp = p.q_sum + ((int64_t)b * p.Hq + h) * D + d;
    const float v = (p.reset ? 0.f : *qsp) + qn;
    *qsp = v;
    qs[g][d] = v;
  }
  for (int c = tid; c < hid; c += 256) wo[c] = p.w_out[c];
  __syncthreads();
  float* ukb = p.uk + ((int64_t)b * p.Hkv + kvh) * p.uk_stride;
  {
    // Projections. Up to 128 hidden units, two threads per unit, each over half of d
    // (partial sums meet in LDS); above that one thread per unit. The loads of eight d run
    // ahead of their FMAs.
    const int per = hid <= 128 ? 128 : 256;
    const int nsp = 256 / per;
    const int c = tid % per, sp = tid / per;
    const int d0 = sp * D / nsp, d1 = (sp + 1) * D / nsp;
    float vk = 0.f;
    float acc[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) acc[g] = 0.f;
    if (c < hid) {
#pragma unroll 8
      for (int d = d0; d < d1; ++d) {
        const float wk = p.wk_t[(int64_t)d * hid + c];
        const float wq = p.wq_t[(int64_t)d * hid + c];
        vk = fmaf(ks[d], wk, vk);
#pragma unroll
        for (int g = 0; g < MG; ++g)
          acc[g] = fmaf(qs[g][d], wq, acc[g]);
      }
    }
    if (nsp == 2 && sp == 1 && c < hid) {
      vrow[c] = vk;
#pragma unroll
      for (int g = 0; g < MG; ++g)
        u[g][c] = acc[g];
    }
    __syncthreads();
    if (sp == 0 && c < hid) {
      if (nsp == 2) {
        vk += vrow[c];
#pragma unroll
        for (int g = 0; g < MG; ++g)
          acc[g] += u[g][c];
      }
      vrow[c] = vk;
      ukb[(int64_t)p.row * hid + c] = vk;
      const float bias = p.b_in[c];
#pragma unroll
      for (int g = 0; g < MG; ++g)
        u[g][c] = acc[g] + bias;
    }
  }
  __syncthreads();
  const int nbk = p.row + 1;
  unsigned int active = 0;
  for (int j = tid; j < nbk; j += 256) {
    float acc[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) acc[g] = 0.f;
    // Block `row` was stored above by this workgroup (visible after the barrier), so every
    // key block is read from the kept units with plain global loads.
    const float* vj = ukb + (int64_t)j * hid;
#pragma unroll 8
    for (int c = 0; c < hid; c += 4) {
      const f32x4_t v4 = *(const f32x4_t*)(vj + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float w = wo[c + e];
#pragma unroll
        for (int g = 0; g < MG; ++g)
          acc[g] = fmaf(w, fmaxf(u[g][c + e] + v4[e], 0.f), acc[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      if (g >= p.G) break;
      const int h = h0 + g;
      const float sv = 1.f / (1.f + expf(-acc[g]));
      const bool on = sv >= p.tau[h] || (p.force_diag && j == p.row);
      const int64_t o = ((int64_t)b * p.Hq + h) * nbk + j;
      p.soft[o] = sv;
      p.mask[o] = on ? 1 : 0;
      active += on ? 1u : 0u;
    }
  }
  const float tot = wave_sum((float)active);
  if (lane == 0) wave_count[wave] = (unsigned int)(tot + 0.5f);
  __syncthreads();
  if (tid == 0) {
    const unsigned int t = (wave_count[0] + wave_count[1]) + (wave_count[2] + wave_count[3]);
    if (t && p.counter) atomicAdd(p.counter, (unsigned long long)t);
  }
}

__global__ void gate_counter_reset_kernel(unsigned long long* counter) {
  if (threadIdx.x == 0) *counter = 0ull;
}

// ---------------------------------------------------------------------------------------
// Backward of the pairwise MLP (gate training).
//
// With u_i = W_q qbar_i + b_in, v_j = W_k kbar_j, pre_ijc = u_ic + v_jc and
// soft_ij = sigmoid(w . relu(pre_ij)) (0 above the block diagonal when causal), the
// gradient G = dL/dsoft gives g_ij = G_ij soft_ij (1 - soft_ij) (0 where soft was zeroed),
// and
//   dL/dw_c   = sum_ij g_ij relu(pre_ijc)
//   dL/du_ic  = w_c sum_j g_ij [pre_ijc > 0]
//   dL/dv_jc  = w_c sum_i g_ij [pre_ijc > 0].
// A workgroup takes a 32 x 32 tile of pairs of one (batch, head) and writes the tile's
// partial sums without the w_c factor: S_u[i][c] = sum over the tile's j, S_v[j][c] over
// its i, S_w[c] over the tile. Partial buffers (fp32, every element written, zeros for
// tiles wholly above the diagonal):
//   du_part [tiles][B][Hq][NB][hidden]  (indexed by the key tile)
//   dv_part [tiles][B][Hq][NB][hidden]  (indexed by the query tile)
//   dw_part [B * Hq * tiles * tiles][hidden]
// The caller sums them and applies w (deterministic: no atomics).
// ---------------------------------------------------------------------------------------
constexpr int kBwdTile = 32;
constexpr int kBwdHC = 64;  // hidden units staged per round

struct GateBwdParams {
  const float* uq;
  const float* uk;
  const float* soft;       // [B, Hq, NB, NB]
  const float* grad_soft;  // [B, Hq, NB, NB]
  float* du_part;
  float* dv_part;
  float* dw_part;
  int B, Hq, Hkv, G, NB, hidden, causal, tiles;
};

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
gate_pairwise_bwd_kernel(const GateBwdParams p) {
  __shared__ float g_t[kBwdTile][kBwdTile + 1];
  __shared__ float uq_s[kBwdTile][kBwdHC + 1];
  __shared__ float uk_s[kBwdTile][kBwdHC + 1];

  const int tid = threadIdx.x;
  const int per_head = p.tiles * p.tiles;
  const int64_t bh = blockIdx.x / per_head;
  const int t2 = (int)(blockIdx.x % per_head);
  const int it = t2 / p.tiles, jt = t2 % p.tiles;
  const int i0 = it * kBwdTile, j0 = jt * kBwdTile;
  const int b = (int)(bh / p.Hq);
  const int h = (int)(bh % p.Hq);
  const int kvh = h / p.G;
  const int64_t plane = (int64_t)p.B * p.Hq * p.NB * p.hidden;
  float* du_out = p.du_part + jt * plane + (bh * p.NB) * (int64_t)p.hidden;
  float* dv_out = p.dv_part + it * plane + (bh * p.NB) * (int64_t)p.hidden;
  float* dw_out = p.dw_part + (int64_t)blockIdx.x * p.hidden;
  const int rows_i = min(kBwdTile, p.NB - i0), rows_j = min(kBwdTile, p.NB - j0);

  if (p.causal && j0 > i0 + kBwdTile - 1) {
    // Wholly above the diagonal: every g is zero.
    for (int e = tid; e < rows_i * p.hidden; e += 256) du_out[(int64_t)i0 * p.hidden + e] = 0.f;
    for (int e = tid; e < rows_j * p.hidden; e += 256) dv_out[(int64_t)j0 * p.hidden + e] = 0.f;
    for (int e = tid; e < p.hidden; e += 256) dw_out[e] = 0.f;
    return;
  }
  const int64_t sbase = bh * (int64_t)p.NB * p.NB;
  for (int e = tid; e < kBwdTile * kBwdTile; e += 256) {
    const int ii = e / kBwdTile, jj = e % kBwdTile;
    const int i = i0 + ii, j = j0 + jj;
    float g = 0.f;
    if (i < p.NB && j < p.NB && !(p.causal && j > i)) {
      const int64_t o = sbase + (int64_t)i * p.NB + j;
      const float sv = p.soft[o];
      g = p.grad_soft[o] * sv * (1.f - sv);
    }
    g_t[ii][jj] = g;
  }

  const float* uq = p.uq + (bh * p.NB) * (int64_t)p.hidden;
  const float* uk = p.uk + (((int64_t)b * p.Hkv + kvh) * p.NB) * (int64_t)p.hidden;
  const int r = tid % kBwdTile;       // row (pass A) / column (pass B) of this thread
  const int ug = tid / kBwdTile;      // unit group: units 8*ug .. 8*ug+7 of a staged round
  for (int c0 = 0; c0 < p.hidden; c0 += kBwdHC) {
    const int hc = min(kBwdHC, p.hidden - c0);
    __syncthreads();  // g_t written (first round); previous round's reads done
    for (int e = tid; e < kBwdTile * kBwdHC; e += 256) {
      const int rr = e / kBwdHC, cc = e % kBwdHC;
      const bool okc = cc < hc;
      uq_s[rr][cc] = (okc && rr < rows_i) ? uq[(int64_t)(i0 + rr) * p.hidden + c0 + cc] : 0.f;
      uk_s[rr][cc] = (okc && rr < rows_j) ? uk[(int64_t)(j0 + rr) * p.hidden + c0 + cc] : 0.f;
    }
    __syncthreads();
    // Pass A: row i = i0 + r, units c0 + 8ug ..: S_u over the tile's keys and S_w.
    float a[8], su[8], sw[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = uq_s[r][8 * ug + e];
      su[e] = 0.f;
      sw[e] = 0.f;
    }
#pragma unroll 4
    for (int jj = 0; jj < kBwdTile; ++jj) {
      const float g = g_t[r][jj];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pre = a[e] + uk_s[jj][8 * ug + e];
        su[e] += pre > 0.f ? g : 0.f;
        sw[e] = fmaf(g, fmaxf(pre, 0.f), sw[e]);
      }
    }
    if (r < rows_i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + 8 * ug + e;
        if (c < p.hidden) du_out[(int64_t)(i0 + r) * p.hidden + c] = su[e];
      }
    }
    // S_w: sum over the 32 rows, held by the 32 consecutive lanes of this unit group.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = sw[e];
#pragma unroll
      for (int off = 1; off < kBwdTile; off <<= 1) x += __shfl_xor(x, off, kWave);
      sw[e] = x;
    }
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + 8 * ug + e;
        if (c < p.hidden) dw_out[c] = sw[e];
      }
    }
    // Pass B: column j = j0 + r: S_v over the tile's queries.
    float bv[8], sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bv[e] = uk_s[r][8 * ug + e];
      sv[e] = 0.f;
    }
#pragma unroll 4
    for (int ii = 0; ii < kBwdTile; ++ii) {
      const float g = g_t[ii][r];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pre = uq_s[ii][8 * ug + e] + bv[e];
        sv[e] += pre > 0.f ? g : 0.f;
      }
    }
    if (r < rows_j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + 8 * ug + e;
        if (c < p.hidden) dv_out[(int64_t)(j0 + r) * p.hidden + c] = sv[e];
      }
    }
  }
}

}  // namespace tasft

using namespace tasft;

// Compute units of the current device (cached per device).
static int gate_device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Diagnostic switch of tasft_gate_debug_wait_fault: while set, the one-launch gate's key
// workgroups publish nothing and each query workgroup's wait gives up after kGateFaultTicks.
static std::atomic<int> g_gate_wait_fault{0};
constexpr unsigned long long kGateFaultTicks = 2000;  // 20 us

extern "C" int tasft_gate_debug_wait_fault(int enable) {
  g_gate_wait_fault.store(enable ? 1 : 0);
  return kOk;
}

// Bytes of the projected units at the front of the gate workspace, rounded up to 256.
static size_t gate_units_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                               int64_t nb, int64_t hidden) {
  const size_t b = (size_t)(batch * (num_q_heads + num_kv_heads) * nb * hidden) * sizeof(float);
  return (b + 255) & ~(size_t)255;
}

extern "C" size_t tasft_gate_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                             int64_t num_kv_heads, int64_t seq_len,
                                             int64_t head_dim, int64_t block_size,
                                             int64_t hidden) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0 ||
      block_size <= 0 || hidden <= 0)
    return 0;
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  // Projected units, hidden fp32 values per query block and per key block, then (at a
  // 256-byte boundary) one 64-byte completion counter per (b, KV head) for the one-launch
  // gate.
  return gate_units_bytes(batch, num_q_heads, num_kv_heads, nb, hidden) +
         (size_t)(batch * num_kv_heads) * kGateSyncStride * sizeof(unsigned int);
}

extern "C" int tasft_gate_fwd(const void* q, const void* k, const float* w_in, const float* b_in,
                              const float* w_out, const float* thresholds, float* soft_scores,
                              float* logits, uint8_t* hard_mask, unsigned long long* active_count,
                              float* q_means, float* k_means,
                              void* workspace, size_t workspace_bytes, int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                              int64_t head_dim, int64_t block_size, int64_t hidden,
                              const int64_t* q_strides, const int64_t* k_strides, int flags,
                              int dtype, void* stream) {
  if (!q || !k || !w_in || !b_in || !w_out || !thresholds || !soft_scores || !hard_mask ||
      !active_count || !workspace || !q_strides || !k_strides)
    return set_error(kErrInvalidArgument, "gate: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "gate: dtype must be bf16 (0) or fp16 (1), got %d", dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || block_size <= 0 ||
      hidden <= 0)
    return set_error(kErrInvalidArgument, "gate: sizes must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "gate: num_q_heads must be a multiple of num_kv_heads");
  if (head_dim % 8 != 0 || head_dim > kGateMaxD || head_dim <= 0)
    return set_error(kErrUnsupported, "gate: head_dim must be a multiple of 8 and at most %d, got %lld",
                     kGateMaxD, (long long)head_dim);
  if (!strides_nonneg(q_strides, 4) || !strides_nonneg(k_strides, 4))
    return set_error(kErrInvalidArgument, "gate: strides must be non-negative");
  if (q_strides[3] != 1 || k_strides[3] != 1)
    return set_error(kErrInvalidArgument, "gate: head_dim must be the contiguous dimension");
  for (int j = 0; j < 3; ++j)
    if (q_strides[j] % 8 != 0 || k_strides[j] % 8 != 0)
      return set_error(kErrInvalidArgument, "gate: strides must be multiples of 8 elements");
  if ((((uintptr_t)q) & 15u) || (((uintptr_t)k) & 15u) || (((uintptr_t)w_in) & 15u))
    return set_error(kErrInvalidArgument, "gate: q, k and w_in must be 16-byte aligned");
  const size_t need = tasft_gate_workspace_bytes(batch, num_q_heads, num_kv_heads, seq_len,
                                                 head_dim, block_size, hidden);
  if (workspace_bytes < need)
    return set_error(kErrWorkspace, "gate: workspace too small: need %zu bytes, got %zu", need,
                     workspace_bytes);
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  const int64_t chunks = (nb + kPoolBlocks - 1) / kPoolBlocks;
  const int64_t tiles = (nb + kPairTile - 1) / kPairTile;
  if (batch * (num_q_heads + num_kv_heads) * chunks > 0x7fffffffLL ||
      batch * num_q_heads * tiles * tiles > 0x7fffffffLL || seq_len > 0x3fffffffLL)
    return set_error(kErrUnsupported, "gate: problem too large for one launch");

  GatePoolParams pp;
  pp.q = (const uint16_t*)q;
  pp.k = (const uint16_t*)k;
  pp.w_in = w_in;
  pp.b_in = b_in;
  pp.uq = (float*)workspace;
  pp.uk = pp.uq + batch * num_q_heads * nb * hidden;
  pp.qmeans = q_means;
  pp.kmeans = k_means;
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

  pp.wg0 = 0;
  pp.rotate = 0;

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
  qp.NBq = pp.NB;
  qp.NBk = pp.NB;
  qp.row0 = 0;
  qp.hidden = pp.hidden;
  qp.causal = (flags & 1) ? 1 : 0;
  qp.force_diag = (flags & 2) ? 1 : 0;
  qp.tiles_q = (int)tiles;
  qp.tiles_k = (int)tiles;
  qp.uk_bh_stride = nb * hidden;

  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  // The streaming pool's 32-bit row offsets reach the end of a chunk's last load group.
  const bool fast = (block_size == 32 || block_size == 64 || block_size == 128) &&
                    (head_dim == 64 || head_dim == 128) &&
                    std::max<int64_t>(seq_len, kFusePB * block_size) *
                            std::max(q_strides[2], k_strides[2]) * 2 < 0x7fffffffLL;
  if (fast) {
    const int64_t fchunks = (nb + kFusePB - 1) / kFusePB;
    // Block 64 with hidden a multiple of kFuseHid, at most kFuseMaxHid: the whole gate in
    // gate_fused64_kernel. Otherwise one launch pools and projects Q and K, and
    // gate_pairwise_kernel follows.
    const bool fused = block_size == 64 && hidden % kFuseHid == 0 && hidden <= kFuseMaxHid;
    if (fused) {
      // One launch: key chunks, then query chunks (gate_fused64_kernel), after the
      // completion counters and the active count are zeroed.
      pp.rotate = 1;
      GateSync sy;
      sy.done = (unsigned int*)((uint8_t*)workspace +
                                gate_units_bytes(batch, num_q_heads, num_kv_heads, nb, hidden));
      sy.wait_ticks = g_gate_wait_fault ? kGateFaultTicks : kGateWaitTicks;
      sy.skip_publish = g_gate_wait_fault ? 1 : 0;
      hipLaunchKernelGGL(gate_sync_reset_kernel, dim3(1), dim3(256), 0, s, sy.done,
                         (int)(batch * num_kv_heads), active_count);
      const dim3 g((unsigned)(batch * (num_q_heads + num_kv_heads) * fchunks));
      if (head_dim == 128 && dtype == kF16)
        hipLaunchKernelGGL((gate_fused64_kernel<128, kF16>), g, dim3(256), 0, s, pp, qp, sy);
      else if (head_dim == 128)
        hipLaunchKernelGGL((gate_fused64_kernel<128, kBf16>), g, dim3(256), 0, s, pp, qp, sy);
      else if (dtype == kF16)
        hipLaunchKernelGGL((gate_fused64_kernel<64, kF16>), g, dim3(256), 0, s, pp, qp, sy);
      else
        hipLaunchKernelGGL((gate_fused64_kernel<64, kBf16>), g, dim3(256), 0, s, pp, qp, sy);
      if ((err = hipGetLastError()) != hipSuccess)
        return set_error(kErrLaunch, "gate: fused launch failed: %s", hipGetErrorString(err));
      return kOk;
    }
    const dim3 g1((unsigned)(batch * (num_q_heads + num_kv_heads) * fchunks));
    if (block_size == 32) {
      if (head_dim == 128 && dtype == kF16)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kF16, 32>), g1, dim3(256), 0, s, pp);
      else if (head_dim == 128)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kBf16, 32>), g1, dim3(256), 0, s, pp);
      else if (dtype == kF16)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kF16, 32>), g1, dim3(256), 0, s, pp);
      else
        hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kBf16, 32>), g1, dim3(256), 0, s, pp);
    } else if (block_size == 128) {
      // Blocks 32 and 128: the same streaming pool, then gate_pairwise_kernel.
      if (head_dim == 128 && dtype == kF16)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kF16, 128>), g1, dim3(256), 0, s, pp);
      else if (head_dim == 128)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kBf16, 128>), g1, dim3(256), 0, s, pp);
      else if (dtype == kF16)
        hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kF16, 128>), g1, dim3(256), 0, s, pp);
      else
        hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kBf16, 128>), g1, dim3(256), 0, s, pp);
    } else if (head_dim == 128 && dtype == kF16)
      hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kF16>), g1, dim3(256), 0, s, pp);
    else if (head_dim == 128)
      hipLaunchKernelGGL((gate_pool_proj64_kernel<128, kBf16>), g1, dim3(256), 0, s, pp);
    else if (dtype == kF16)
      hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kF16>), g1, dim3(256), 0, s, pp);
    else
      hipLaunchKernelGGL((gate_pool_proj64_kernel<64, kBf16>), g1, dim3(256), 0, s, pp);
    if ((err = hipGetLastError()) != hipSuccess)
      return set_error(kErrLaunch, "gate: pool launch failed: %s", hipGetErrorString(err));
  } else {
    const dim3 g1((unsigned)(batch * (num_q_heads + num_kv_heads) * chunks));
    if (dtype == kF16)
      hipLaunchKernelGGL(gate_pool_project_kernel<kF16>, g1, dim3(256), 0, s, pp);
    else
      hipLaunchKernelGGL(gate_pool_project_kernel<kBf16>, g1, dim3(256), 0, s, pp);
    if ((err = hipGetLastError()) != hipSuccess)
      return set_error(kErrLaunch, "gate: pool launch failed: %s", hipGetErrorString(err));
  }

  const int64_t grid2 = batch * num_q_heads * tiles * tiles;
  hipLaunchKernelGGL(gate_pairwise_kernel, dim3((unsigned)grid2), dim3(256), 0, s, qp);
  if ((err = hipGetLastError()) != hipSuccess)
    return set_error(kErrLaunch, "gate: pairwise launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" size_t tasft_gate_bwd_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                                 int64_t seq_len, int64_t block_size,
                                                 int64_t hidden) {
  if (batch <= 0 || num_q_heads <= 0 || seq_len <= 0 || block_size <= 0 || hidden <= 0) return 0;
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  const int64_t tiles = (nb + kBwdTile - 1) / kBwdTile;
  const int64_t plane = batch * num_q_heads * nb * hidden;
  return (size_t)(2 * tiles * plane + batch * num_q_heads * tiles * tiles * hidden) * sizeof(float);
}

extern "C" int tasft_gate_bwd(const float* soft_scores, const float* grad_soft,
                              const void* fwd_workspace, size_t fwd_workspace_bytes,
                              float* partials, size_t partials_bytes, int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                              int64_t block_size, int64_t hidden, int flags, void* stream) {
  if (!soft_scores || !grad_soft || !fwd_workspace || !partials)
    return set_error(kErrInvalidArgument, "gate_bwd: null pointer argument");
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || block_size <= 0 ||
      hidden <= 0)
    return set_error(kErrInvalidArgument, "gate_bwd: sizes must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "gate_bwd: num_q_heads must be a multiple of num_kv_heads");
  const size_t fwd_need = tasft_gate_workspace_bytes(batch, num_q_heads, num_kv_heads, seq_len, 8,
                                                     block_size, hidden);
  if (fwd_workspace_bytes < fwd_need)
    return set_error(kErrWorkspace, "gate_bwd: forward workspace too small: need %zu bytes, got %zu",
                     fwd_need, fwd_workspace_bytes);
  const size_t need = tasft_gate_bwd_workspace_bytes(batch, num_q_heads, seq_len, block_size, hidden);
  if (partials_bytes < need)
    return set_error(kErrWorkspace, "gate_bwd: partials buffer too small: need %zu bytes, got %zu",
                     need, partials_bytes);
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  const int64_t tiles = (nb + kBwdTile - 1) / kBwdTile;
  if (batch * num_q_heads * tiles * tiles > 0x7fffffffLL)
    return set_error(kErrUnsupported, "gate_bwd: problem too large for one launch");
  GateBwdParams bp;
  bp.uq = (const float*)fwd_workspace;
  bp.uk = bp.uq + batch * num_q_heads * nb * hidden;
  bp.soft = soft_scores;
  bp.grad_soft = grad_soft;
  const int64_t plane = batch * num_q_heads * nb * hidden;
  bp.du_part = partials;
  bp.dv_part = partials + tiles * plane;
  bp.dw_part = partials + 2 * tiles * plane;
  bp.B = (int)batch;
  bp.Hq = (int)num_q_heads;
  bp.Hkv = (int)num_kv_heads;
  bp.G = (int)(num_q_heads / num_kv_heads);
  bp.NB = (int)nb;
  bp.hidden = (int)hidden;
  bp.causal = (flags & 1) ? 1 : 0;
  bp.tiles = (int)tiles;
  hipLaunchKernelGGL(gate_pairwise_bwd_kernel, dim3((unsigned)(batch * num_q_heads * tiles * tiles)),
                     dim3(256), 0, (hipStream_t)stream, bp);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate_bwd: launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" int tasft_gate_rows_fwd(const float* uq, const float* uk, const float* w_out,
                                   const float* thresholds, float* soft_scores, float* logits,
                                   uint8_t* hard_mask, unsigned long long* active_count,
                                   int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                   int64_t rows, int64_t key_blocks, int64_t row0, int64_t hidden,
                                   int64_t uk_head_stride, int flags, void* stream) {
  if (!uq || !uk || !w_out || !thresholds || !soft_scores || !hard_mask || !active_count)
    return set_error(kErrInvalidArgument, "gate_rows: null pointer argument");
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || rows <= 0 || key_blocks <= 0 ||
      hidden <= 0 || row0 < 0)
    return set_error(kErrInvalidArgument, "gate_rows: sizes must be positive (row0 >= 0)");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "gate_rows: num_q_heads must be a multiple of num_kv_heads");
  if ((((uintptr_t)uq) & 15u) || (((uintptr_t)uk) & 15u))
    return set_error(kErrInvalidArgument, "gate_rows: uq and uk must be 16-byte aligned");
  if (uk_head_stride < key_blocks * hidden || uk_head_stride % 4 != 0 || hidden % 4 != 0)
    return set_error(kErrInvalidArgument,
                     "gate_rows: uk_head_stride must be >= key_blocks * hidden, and it and hidden "
                     "multiples of 4");
  const int64_t tq = (rows + kPairTile - 1) / kPairTile;
  const int64_t tk = (key_blocks + kPairTile - 1) / kPairTile;
  if (batch * num_q_heads * tq * tk > 0x7fffffffLL || row0 + rows > 0x7fffffffLL)
    return set_error(kErrUnsupported, "gate_rows: problem too large for one launch");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(gate_counter_reset_kernel, dim3(1), dim3(64), 0, s, active_count);
  GatePairParams qp;
  qp.uq = uq;
  qp.uk = uk;
  qp.w_out = w_out;
  qp.tau = thresholds;
  qp.soft = soft_scores;
  qp.logits = logits;
  qp.mask = hard_mask;
  qp.counter = active_count;
  qp.B = (int)batch;
  qp.Hq = (int)num_q_heads;
  qp.Hkv = (int)num_kv_heads;
  qp.G = (int)(num_q_heads / num_kv_heads);
  qp.NBq = (int)rows;
  qp.NBk = (int)key_blocks;
  qp.row0 = (int)row0;
  qp.hidden = (int)hidden;
  qp.causal = (flags & 1) ? 1 : 0;
  qp.force_diag = (flags & 2) ? 1 : 0;
  qp.tiles_q = (int)tq;
  qp.tiles_k = (int)tk;
  qp.uk_bh_stride = uk_head_stride;
  hipLaunchKernelGGL(gate_pairwise_kernel, dim3((unsigned)(batch * num_q_heads * tq * tk)), dim3(256),
                     0, s, qp);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate_rows: launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" int tasft_gate_decode_rows_fwd(
    const void* q_new, const void* k_new, const int64_t* q_strides, const int64_t* k_strides,
    float* q_sum, float* k_sum, float* uk, int64_t uk_head_stride, const float* wq_t,
    const float* wk_t, const float* b_in, const float* w_out, const float* thresholds,
    float* soft_scores, uint8_t* hard_mask, unsigned long long* active_count, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t hidden, int64_t row,
    int reset_sums, int flags, int dtype, void* stream) {
  if (!q_new || !k_new || !q_strides || !k_strides || !q_sum || !k_sum || !uk || !wq_t ||
      !wk_t || !b_in || !w_out || !thresholds || !soft_scores || !hard_mask)
    return set_error(kErrInvalidArgument, "gate_decode_rows: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "gate_decode_rows: dtype must be bf16 (0) or fp16 (1), got %d",
                     dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || hidden <= 0 ||
      row < 0)
    return set_error(kErrInvalidArgument, "gate_decode_rows: sizes must be positive (row >= 0)");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument,
                     "gate_decode_rows: num_q_heads must be a multiple of num_kv_heads");
  const int64_t G = num_q_heads / num_kv_heads;
  if (G > kRowMaxG || head_dim > kGateMaxD || hidden > kRowMaxHid || hidden % 4 != 0)
    return set_error(kErrUnsupported,
                     "gate_decode_rows: needs at most %d query heads per KV head, head_dim <= %d "
                     "and hidden <= %d, a multiple of 4 (got %lld, %lld, %lld)",
                     kRowMaxG, kGateMaxD, kRowMaxHid, (long long)G, (long long)head_dim,
                     (long long)hidden);
  if (uk_head_stride < (row + 1) * hidden || uk_head_stride % 4 != 0 ||
      (((uintptr_t)uk) & 15u))
    return set_error(kErrInvalidArgument,
                     "gate_decode_rows: uk_head_stride must hold row + 1 blocks and be a multiple "
                     "of 4, uk 16-byte aligned");
  if (!strides_nonneg(q_strides, 2) || !strides_nonneg(k_strides, 2))
    return set_error(kErrInvalidArgument, "gate_decode_rows: strides must be non-negative");
  if (batch * num_kv_heads > 0x7fffffffLL || row >= 0x3fffffffLL)
    return set_error(kErrUnsupported, "gate_decode_rows: problem too large for one launch");
  GateDecodeRowParams rp;
  rp.q_new = (const uint16_t*)q_new;
  rp.k_new = (const uint16_t*)k_new;
  for (int j = 0; j < 2; ++j) {
    rp.sq[j] = q_strides[j];
    rp.sk[j] = k_strides[j];
  }
  rp.q_sum = q_sum;
  rp.k_sum = k_sum;
  rp.uk = uk;
  rp.uk_stride = uk_head_stride;
  rp.wq_t = wq_t;
  rp.wk_t = wk_t;
  rp.b_in = b_in;
  rp.w_out = w_out;
  rp.tau = thresholds;
  rp.soft = soft_scores;
  rp.mask = hard_mask;
  rp.counter = active_count;
  rp.B = (int)batch;
  rp.Hq = (int)num_q_heads;
  rp.Hkv = (int)num_kv_heads;
  rp.G = (int)G;
  rp.D = (int)head_dim;
  rp.hidden = (int)hidden;
  rp.row = (int)row;
  rp.reset = reset_sums ? 1 : 0;
  rp.force_diag = (flags & 2) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (active_count) hipLaunchKernelGGL(gate_counter_reset_kernel, dim3(1), dim3(64), 0, s, active_count);
  const dim3 grid((unsigned)(batch * num_kv_heads));
  auto launch = [&](auto mg) {
    constexpr int MG = decltype(mg)::value;
    if (dtype == kF16)
      hipLaunchKernelGGL((gate_decode_row_kernel<kF16, MG>), grid, dim3(256), 0, s, rp);
    else
      hipLaunchKernelGGL((gate_decode_row_kernel<kBf16, MG>), grid, dim3(256), 0, s, rp);
  };
  if (G == 1)
    launch(std::integral_constant<int, 1>());
  else if (G == 2)
    launch(std::integral_constant<int, 2>());
  else if (G <= 4)
    launch(std::integral_constant<int, 4>());
  else
    launch(std::integral_constant<int, 8>());
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate_decode_rows: launch failed: %s", hipGetErrorString(err));
  return kOk;
}
