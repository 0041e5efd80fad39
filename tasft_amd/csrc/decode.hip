// Split-K block-sparse decode for gfx950 (memory bound).
//
// The reference has no sparse decode: its vLLM patch hands decode to the dense
// PagedAttention (tasft/inference/vllm_patch.py:189-196, 215-252) and the HF path
// rejects S_q != S_k (tasft/modules/attn_gate.py:216-221). The semantics implemented
// here are the closed form of the prefill kernel's last query row
// (tasft/kernels/block_sparse_fa.py:192-269): for one new query token per sequence,
//   o[b, h] = softmax(q[b, h] . K_sel^T * scale) . V_sel
// over the tokens < kv_len of the key blocks selected for query head h; a head with no
// selected block outputs 0.
//
// Data path. A workgroup owns (batch b, KV head kvh, split s). For blocks of up to 64
// keys the split is a share of the selected blocks: the blocks selected by any of the G
// query heads of kvh are numbered in block order and split s takes entries
// [s*n/P, (s+1)*n/P), so the splits of a row do equal work. (For 128-key blocks it is
// the contiguous range of key blocks [s*NB/P, (s+1)*NB/P).) Its 4 waves take the
// blocks round-robin. Each selected KV block is read from HBM once per KV
// head, however many query heads chose it; all its K and V loads are issued together.
// QK^T runs on MFMA (v_mfma_f32_32x32x16_bf16, or _f16 for fp16 inputs; K is loaded straight into the A-operand
// layout, the G query heads are the N columns), PV on the VALU. Partial
// (max, sum, output) triples per (b, h, split) go to a caller-provided workspace and a
// second kernel merges them.
#include "common.h"

#include <mutex>

#include "../../include/tasft_amd.h"

namespace tasft {

constexpr int kDecodeMaxG = 8;    // query heads per KV head handled by one workgroup
constexpr int kDecodeWaves = 4;
constexpr int kDecodeMaxRange = 1024;  // key blocks per split (mask bytes staged in LDS)

struct DecodeParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  const uint8_t* mask;     // [B, Hq, 1, NB]
  const int32_t* kv_lens;  // [B] or null
  float* ws_o;             // [B, Hq, P, D]
  float* ws_ml;            // [B, Hq, P, 2]
  int64_t sq[2], sk[3], sv[3], so[2], sm[3];
  int B, Hq, Hkv, G, S_kv, NB, P;
  float scale_log2;
  // Paged cache (kernels instantiated with PAGED): K/V are page pools whose strides sk, sv
  // are (page, head, token); token t of sequence b lives in page
  // block_table[b * bt_stride + t / page_size], row t % page_size.
  // Page ids are clamped to [0, num_pages): a bad table entry reads a wrong page of the
  // pool, never memory outside it.
  const int32_t* block_table;
  int64_t bt_stride;
  int page_size;
  int num_pages;
  // Mask index shift: key block t reads mask entry t >> mshift. 1 runs a block-128 mask on
  // the block-64 kernel (a 128-key block is its two 64-key halves); 0 otherwise.
  int mshift;
};

// Raw buffer resource (stride 0) over `bytes` bytes starting at `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t decode_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n, 0x00020000);
}

// s_waitcnt immediate waiting until at most n vector-memory operations are outstanding
// (expcnt and lgkmcnt left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One 16-byte-per-lane DMA (buffer_load ... lds) of 1 KB into LDS at `dst`. V is read
// once per call, so the DMA is non-temporal (cache policy nt): measured 143 against 159 us
// at config 3. The same bit on the K loads into registers measured slower (173-184 us).
constexpr int kStreamNT = 2;
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (TASFT_LDS void*)dst, 16, voff, 0, 0, kStreamNT);
}

__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// SUB keys (<= 64) of one KV block are processed at a time; a block of BS keys is
// BS/SUB sub-blocks. MG >= G is the head count the loops are unrolled for (padding heads
// carry zero probability). Up to four heads run two waves per SIMD (at most 256
// registers each, two workgroups per CU). Five to eight heads need more than that: built
// for two waves per SIMD they spilled about 120 bytes per lane to scratch inside the
// block loop, so they run one wave per SIMD (up to 512 registers, one workgroup per CU).
template <int BS, int D, int MG, bool PAGED, int DT>
__global__ void __launch_bounds__(kDecodeWaves * kWave, MG == 8 ? 1 : 2)
bsfa_decode_split_kernel(const DecodeParams p) {
  static_assert(!PAGED || BS <= 64, "paged caches use the one-sub-block path");
  constexpr int SUB = BS < 64 ? BS : 64;
  constexpr int NSUB = BS / SUB;
  constexpr int KT = SUB / 32;        // 32-key MFMA tiles per sub-block
  constexpr int KSTEPS = D / 16;      // MFMA k-steps over the head dim
  constexpr int DOCT = D / 8;         // 16-byte chunks per row
  constexpr int KG = kWave / DOCT;    // key groups in the PV phase
  constexpr int VPL = SUB / KG;       // V rows per lane per sub-block

  constexpr int VTILE = SUB * D * 2;  // bytes of one sub-block of V
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[kDecodeWaves][VTILE];  // per-wave V tile
  __shared__ uint8_t hb[kDecodeMaxRange];  // head bits per block of the range / per entry
  __shared__ int sel[kDecodeMaxRange];      // selected blocks (range offsets / block indices)
  __shared__ int wsum[kDecodeWaves];
  __shared__ float p_lds[kDecodeWaves][SUB * MG + kWave];     // probabilities (+ dummy slots)
  __shared__ float a_lds[kDecodeWaves][MG];                   // rescale factor per head
  __shared__ float comb_ml[kDecodeWaves][MG][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop state
  const int col = lane & 31;   // QK layout: query head of this lane
  const int half = lane >> 5;
  const int G = p.G;

  const int64_t item = blockIdx.x;
  const int s = (int)(item % p.P);
  const int64_t bk = item / p.P;
  const int b = (int)(bk / p.Hkv);
  const int kvh = (int)(bk % p.Hkv);
  const int h0 = kvh * G;

  const int kv_len = p.kv_lens ? min(max(p.kv_lens[b], 0), p.S_kv) : p.S_kv;
  const int nb_valid = (kv_len + BS - 1) / BS;
  const int lo = (int)(((int64_t)s * p.NB) / p.P);
  const int hi = min((int)(((int64_t)(s + 1) * p.NB) / p.P), nb_valid);
  const int range = max(hi - lo, 0);

  // Mask bits of key block t for the group's heads.
  const uint8_t* mbase = p.mask + b * p.sm[0] + (int64_t)h0 * p.sm[1];
  auto head_bits = [&](int t) -> uint32_t {
    uint32_t bitsv = 0;
#pragma unroll
    for (int gg = 0; gg < MG; ++gg)
      if (gg < G && mbase[(int64_t)gg * p.sm[1] + (int64_t)(t >> p.mshift) * p.sm[2]]) bitsv |= 1u << gg;
    return bitsv;
  };
  if constexpr (NSUB != 1) {
    // Mask bytes of the range for the group's heads, one round trip.
    for (int t = tid; t < range; t += kDecodeWaves * kWave) hb[t] = (uint8_t)head_bits(lo + t);
  }

  // Q^T as the MFMA B operand: lane (col, half) holds head h0+col, head dims
  // ks*16 + half*8 .. +7. Columns >= G are zero.
  u32x4_t qf[KSTEPS];
  {
    const bool hv = col < G;
    const uint16_t* qrow = p.q + b * p.sq[0] + (int64_t)(h0 + (hv ? col : 0)) * p.sq[1];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4_t val = {0u, 0u, 0u, 0u};
      if (hv) val = *(const u32x4_t*)(qrow + ks * 16 + half * 8);
      qf[ks] = val;
    }
  }
  __syncthreads();

  const uint16_t* kbase = PAGED ? p.k + kvh * p.sk[1] : p.k + b * p.sk[0] + kvh * p.sk[1];
  const uint16_t* vbase = PAGED ? p.v + kvh * p.sv[1] : p.v + b * p.sv[0] + kvh * p.sv[1];
  const int ks2 = (int)p.sk[2], vs2 = (int)p.sv[2];  // row strides (elements)

  // QK-layout state of this lane's head (identical in lanes l and l^32).
  float m_run = -INFINITY, l_run = 0.f;
  // PV-layout accumulators: lane (kg, dc) holds head dims dc*8..+7 of every head.
  const int dc = lane % DOCT;
  const int kg = lane / DOCT;
  float oacc[MG][8];
#pragma unroll
  for (int gg = 0; gg < MG; ++gg)
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[gg][i] = 0.f;
  // Per-lane byte offsets inside a sub-block: K row `col` (A-operand layout); for the V
  // DMA, lane l of unit u fetches byte u*1024 + 16*l of the row-major tile.
  const int k_voff = (col * ks2 + half * 8) * 2;
  // Unit u covers rows u*RPU .. u*RPU+RPU-1 (RPU = 1024 / row bytes): a per-lane base
  // plus u * v_unit_stride. The whole offset stays in the per-lane (VGPR) offset, which
  // the buffer range check covers, so rows past kv_len read as zeros.
  constexpr int RPU = 1024 / (D * 2);
  const int v_dma_base = (lane / (kWave / RPU)) * vs2 * 2 + (lane % (kWave / RPU)) * 16;
  const int v_unit_stride = RPU * vs2 * 2;
  // Where this lane's probabilities go in p_lds (lanes of padding heads: a dummy slot).
  const bool pcol = col < MG;

  if constexpr (NSUB == 1) {
    // Selected blocks of the range, compacted once (wave 0), then taken round-robin by
    // the waves. Each wave keeps the next block's loads in flight: its K loads are issued
    // into the K registers as soon as the S MFMAs have read them, and its V DMA into the
    // wave's V tile as soon as the PV product has read it.
    // Balanced splits: the blocks selected by any head of the group are numbered over
    // the whole row in block order, and split s takes entries [s*n/P, (s+1)*n/P) (a
    // range split would give the splits of one row unequal counts). Two passes over the
    // row's mask bytes: count, then gather this split's (block, head bits) entries.
    // With one split the count pass is skipped: the split takes every entry.
    constexpr int NT = kDecodeWaves * kWave;
    int start = 0, end = 0x7fffffff;
    if (p.P > 1) {
      int cnt = 0;
      for (int t = tid; t < nb_valid; t += NT) cnt += head_bits(t) != 0u ? 1 : 0;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off, kWave);
      if (lane == 0) wsum[wave] = cnt;
      __syncthreads();
      const int n_all = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
      start = (int)(((int64_t)s * n_all) / p.P);
      end = (int)(((int64_t)(s + 1) * n_all) / p.P);
      __syncthreads();  // wsum is rewritten below
    }
    int base = 0;     // entries before this chunk (uniform)
    for (int c0 = 0; c0 < nb_valid && base < end; c0 += NT) {
      const int t = c0 + tid;
      const uint32_t bv = t < nb_valid ? head_bits(t) : 0u;
      const uint64_t bal = __ballot(bv != 0u);
      if (lane == 0) wsum[wave] = __popcll(bal);
      __syncthreads();
      int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
      for (int w = 0; w < wave; ++w) pos += wsum[w];
      if (bv != 0u && pos >= start && pos < end) {
        sel[pos - start] = t;
        hb[pos - start] = (uint8_t)bv;
      }
      base += (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
      __syncthreads();
    }
    // Uniform values (scalar registers) keep the buffer resources scalar.
    const int nsel = __builtin_amdgcn_readfirstlane(min(end, base) - start);
    constexpr int NKL = KT * KSTEPS;  // K load instructions per block
    u32x4_t ka[KT][KSTEPS];
    // Paged cache: lane j < npg of `pgv` holds the page of the block's j-th page-sized
    // piece (one block ahead of use, so its load is covered by the fixed V wait). A block
    // of BS keys starts at row off0 of its first page.
    constexpr int RPU_ = 1024 / (D * 2);
    const int ps = p.page_size;
    const int npg = ps >= BS ? 1 : BS / ps;
    auto load_pg = [&](int kb) -> int {
      const int first = (kb * BS) / ps;
      // Only pages that hold a token below kv_len are read (later entries may not exist).
      const int jmax = (kv_len - 1 - kb * BS + (kb * BS) % ps) / ps;
      const int id = p.block_table[(int64_t)b * p.bt_stride + first + min(lane < npg ? lane : 0, jmax)];
      return min(max(id, 0), p.num_pages - 1);
    };
    auto load_k_paged = [&](int kb, int pgv) {
      const int key0 = kb * BS;
      const int off0 = key0 % ps;
      const int last = kv_len - 1 - key0;  // rows past it read row kv_len-1 (masked)
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2) {
        const int row = min(t2 * 32 + col, last) + off0;
        const int page = __shfl(pgv, row / ps, kWave);
        const uint16_t* src = kbase + (int64_t)page * p.sk[0] + (int64_t)(row % ps) * ks2 + half * 8;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) ka[t2][ks] = *(const u32x4_t*)(src + ks * 16);
      }
    };
    auto dma_v_paged = [&](int kb, int pgv) {
      const int key0 = kb * BS;
      const int off0 = key0 % ps;
#pragma unroll
      for (int u = 0; u < VTILE / 1024; ++u) {
        // Unit u covers rows u*RPU_ .. +RPU_-1 of the block, inside one page (ps % RPU_ == 0).
        const int row = u * RPU_ + off0;
        const int page = __builtin_amdgcn_readlane(pgv, row / ps);
        const int rows = min(RPU_, kv_len - key0 - u * RPU_);
        const __amdgpu_buffer_rsrc_t vr = decode_rsrc(
            vbase + (int64_t)page * p.sv[0] + (int64_t)(row % ps) * vs2, (int64_t)max(rows, 0) * vs2 * 2);
        dma16(vr, v_lds[wave] + u * 1024, v_dma_base);
      }
    };
    auto load_k = [&](int kb, int pgv) {
      if constexpr (PAGED) {
        load_k_paged(kb, pgv);
        return;
      }
      const int key0 = kb * BS;
      const __amdgpu_buffer_rsrc_t kr = decode_rsrc(kbase + (int64_t)key0 * ks2, (int64_t)SUB * ks2 * 2);
      if (key0 + SUB <= kv_len) {
#pragma unroll
        for (int t2 = 0; t2 < KT; ++t2)
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
            ka[t2][ks] = buf_load16(kr, k_voff + ks * 32, t2 * 32 * ks2 * 2);
      } else {
        // Partial last block: K rows past kv_len are replaced by row kv_len-1; their
        // scores are masked to -inf.
        const int last = kv_len - 1 - key0;
#pragma unroll
        for (int t2 = 0; t2 < KT; ++t2) {
          const int row = min(t2 * 32 + col, last);
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
            ka[t2][ks] = buf_load16(kr, (row * ks2 + half * 8) * 2 + ks * 32, 0);
        }
      }
    };
    auto dma_v = [&](int kb, int pgv) {
      if constexpr (PAGED) {
        dma_v_paged(kb, pgv);
        return;
      }
      const int key0 = kb * BS;
      // The resource ends at row kv_len-1, so rows past kv_len arrive as zeros.
      const __amdgpu_buffer_rsrc_t vr =
          decode_rsrc(vbase + (int64_t)key0 * vs2, (int64_t)min(SUB, kv_len - key0) * vs2 * 2);
#pragma unroll
      for (int u = 0; u < VTILE / 1024; ++u) dma16(vr, v_lds[wave] + u * 1024, v_dma_base + u * v_unit_stride);
    };
    int e = wave;
    int pg_n = 0;  // pages of the next block (paged cache)
    if (e < nsel) {
      const int t0 = __builtin_amdgcn_readfirstlane((int)sel[e]);
      const int pg0 = PAGED ? load_pg(t0) : 0;
      if constexpr (PAGED) {
        const int e1 = e + kDecodeWaves;
        pg_n = load_pg(e1 < nsel ? __builtin_amdgcn_readfirstlane((int)sel[e1]) : t0);
      }
      load_k(t0, pg0);
      dma_v(t0, pg0);
    }
    while (e < nsel) {
      const int kb = __builtin_amdgcn_readfirstlane(sel[e]);
      const int key0 = kb * BS;
      const uint32_t hsel = __builtin_amdgcn_readfirstlane((int)hb[e]);
      const bool head_on = col < G && ((hsel >> col) & 1u);
      // S^T = K Q^T: rows = keys, cols = heads.
      f32x16_t sacc[KT];
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2) {
        sacc[t2] = (f32x16_t){};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
          sacc[t2] = mfma16<DT>(ka[t2][ks], qf[ks], sacc[t2]);
      }
      // The next block of this wave: its K loads go out now (the K registers are free).
      const int en = e + kDecodeWaves;
      const bool more = en < nsel;
      const int tn = more ? __builtin_amdgcn_readfirstlane((int)sel[en]) : 0;
      int pg_nn = 0;
      if constexpr (PAGED) {
        // Pages of the block after the next, issued before the next block's K loads so
        // the fixed V wait below also covers them.
        const int enn = en + kDecodeWaves;
        pg_nn = load_pg(enn < nsel ? __builtin_amdgcn_readfirstlane((int)sel[enn]) : kb);
      }
      if (more) load_k(tn, pg_n);
      // Register r of tile t2 holds key t2*32 + 8*(r/4) + 4*half + r%4 of head `col`.
      float mx = -INFINITY;
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + t2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const float x = (head_on && key < kv_len) ? sacc[t2][r] * p.scale_log2 : -INFINITY;
          sacc[t2][r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = pair_max32(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float ls = 0.f;
      float* pw = p_lds[wave];
#pragma unroll
      for (int t2 = 0; t2 < KT; ++t2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e2 = __builtin_amdgcn_exp2f(sacc[t2][r] - m_use);
          ls += e2;
          const int key = t2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          pw[pcol ? key * MG + col : SUB * MG + lane] = e2;
        }
      }
      l_run = l_run * alpha + ls;
      m_run = m_new;
      if (half == 0 && col < MG) a_lds[wave][col] = alpha;
      // p_lds / a_lds / v_lds are private to this wave: wait for this block's V DMA (the
      // next block's K loads, issued after it, may still be in flight), then a wave
      // barrier orders the LDS writes and reads.
      if (more) __builtin_amdgcn_s_waitcnt(vmcnt_imm(NKL));
      else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // PV: oacc[g] = alpha_g * oacc[g] + sum_key p[key][g] * V[key][dc*8..+7].
#pragma unroll
      for (int gg = 0; gg < MG; ++gg) {
        const float a = a_lds[wave][gg];
#pragma unroll
        for (int j = 0; j < 8; ++j) oacc[gg][j] *= a;
      }
#pragma unroll 2
      for (int i = 0; i < VPL; ++i) {
        const int kk = kg + KG * i;
        float vf[8];
        unpack16x8<DT>(*(const u32x4_t*)(v_lds[wave] + kk * (D * 2) + dc * 16), vf);
#pragma unroll
        for (int gg = 0; gg < MG; ++gg) {
          const float pv = pw[kk * MG + gg];
#pragma unroll
          for (int j = 0; j < 8; ++j) oacc[gg][j] = fmaf(pv, vf[j], oacc[gg][j]);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (more) {
        // The DMA writes the V tile through the memory path: every LDS read of it must
        // have returned first.
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        dma_v(tn, pg_n);
      }
      pg_n = pg_nn;
      e = en;
    }
  } else {
  int rank = 0;  // union rank of the next entry in this range (uniform)
  for (int c0 = 0; c0 < range; c0 += kWave) {
    const int t = c0 + lane;
    const uint32_t mybits = t < range ? hb[t] : 0u;
    uint64_t bits = __ballot(mybits != 0);
    while (bits) {
      const int pos = __builtin_ctzll(bits);
      bits &= bits - 1;
      const int e = rank++;
      if ((e & (kDecodeWaves - 1)) != wave) continue;
      const int kb = lo + c0 + pos;
      const uint32_t hsel = __builtin_amdgcn_readlane(mybits, pos);
      const bool head_on = col < G && ((hsel >> col) & 1u);
#pragma unroll 1
      for (int sb = 0; sb < NSUB; ++sb) {
        const int key0 = kb * BS + sb * SUB;
        if (key0 >= kv_len) break;
        // Issue every K (A-operand layout) and V (PV layout) load of the sub-block.
        const __amdgpu_buffer_rsrc_t kr = decode_rsrc(kbase + (int64_t)key0 * ks2, (int64_t)SUB * ks2 * 2);
        // V: DMA into this wave's LDS tile. The resource ends at row kv_len-1, so rows
        // past kv_len (possibly never written) arrive as zeros.
        const __amdgpu_buffer_rsrc_t vr =
            decode_rsrc(vbase + (int64_t)key0 * vs2, (int64_t)min(SUB, kv_len - key0) * vs2 * 2);
#pragma unroll
        for (int u = 0; u < VTILE / 1024; ++u)
          dma16(vr, v_lds[wave] + u * 1024, v_dma_base + u * v_unit_stride);
        u32x4_t ka[KT][KSTEPS];
        if (key0 + SUB <= kv_len) {
#pragma unroll
          for (int t2 = 0; t2 < KT; ++t2)
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
              ka[t2][ks] = buf_load16(kr, k_voff + ks * 32, t2 * 32 * ks2 * 2);
        } else {
          // Partial last sub-block: K rows past kv_len are replaced by row kv_len-1; their
          // scores are masked to -inf.
          const int last = kv_len - 1 - key0;
#pragma unroll
          for (int t2 = 0; t2 < KT; ++t2) {
            const int row = min(t2 * 32 + col, last);
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
              ka[t2][ks] = buf_load16(kr, (row * ks2 + half * 8) * 2 + ks * 32, 0);
          }
        }
        // S^T = K Q^T: rows = keys, cols = heads.
        f32x16_t sacc[KT];
#pragma unroll
        for (int t2 = 0; t2 < KT; ++t2) {
          sacc[t2] = (f32x16_t){};
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
            sacc[t2] = mfma16<DT>(ka[t2][ks], qf[ks], sacc[t2]);
        }
        // Register r of tile t2 holds key t2*32 + 8*(r/4) + 4*half + r%4 of head `col`.
        float mx = -INFINITY;
#pragma unroll
        for (int t2 = 0; t2 < KT; ++t2) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = key0 + t2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            const float x = (head_on && key < kv_len) ? sacc[t2][r] * p.scale_log2 : -INFINITY;
            sacc[t2][r] = x;
            mx = fmaxf(mx, x);
          }
        }
        mx = pair_max32(mx);
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float ls = 0.f;
        float* pw = p_lds[wave];
#pragma unroll
        for (int t2 = 0; t2 < KT; ++t2) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float e2 = __builtin_amdgcn_exp2f(sacc[t2][r] - m_use);
            ls += e2;
            const int key = t2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            pw[pcol ? key * MG + col : SUB * MG + lane] = e2;
          }
        }
        l_run = l_run * alpha + ls;
        m_run = m_new;
        if (half == 0 && col < MG) a_lds[wave][col] = alpha;
        // p_lds / a_lds / v_lds are private to this wave: wait for the V DMA, then a wave
        // barrier orders the LDS writes and reads.
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // PV: oacc[g] = alpha_g * oacc[g] + sum_key p[key][g] * V[key][dc*8..+7].
#pragma unroll
        for (int gg = 0; gg < MG; ++gg) {
          const float a = a_lds[wave][gg];
#pragma unroll
          for (int j = 0; j < 8; ++j) oacc[gg][j] *= a;
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int kk = kg + KG * i;
          float vf[8];
          unpack16x8<DT>(*(const u32x4_t*)(v_lds[wave] + kk * (D * 2) + dc * 16), vf);
#pragma unroll
          for (int gg = 0; gg < MG; ++gg) {
            const float pv = pw[kk * MG + gg];
#pragma unroll
            for (int j = 0; j < 8; ++j) oacc[gg][j] = fmaf(pv, vf[j], oacc[gg][j]);
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }

  }
  // Per wave: reduce the PV partials over key groups and the denominators over the lane
  // pair, then merge the 4 waves. Each wave's partial output goes to its own V tile.
  static_assert(MG * D * 4 <= VTILE, "merge buffer size");
  __builtin_amdgcn_s_waitcnt(0x0f70);  // no V DMA may still target the tile
  const float l_tot = pair_sum32(l_run);
  if (half == 0 && col < MG) {
    comb_ml[wave][col][0] = m_run;
    comb_ml[wave][col][1] = l_tot;
  }
#pragma unroll
  for (int gg = 0; gg < MG; ++gg) {
#pragma unroll
    for (int off = DOCT; off < kWave; off <<= 1)
#pragma unroll
      for (int j = 0; j < 8; ++j) oacc[gg][j] += __shfl_xor(oacc[gg][j], off, 64);
    if (lane < DOCT) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ((float*)v_lds[wave])[gg * D + lane * 8 + j] = oacc[gg][j];
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kDecodeWaves * kWave) {
    const int gg = i / D, d = i % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, comb_ml[w][gg][0]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(comb_ml[w][gg][0] - Mu);
      L += comb_ml[w][gg][1] * f;
      O += ((const float*)v_lds[w])[gg * D + d] * f;
    }
    if (p.P == 1) {
      // One split: this is the whole row, written directly (no combine pass). An empty row
      // has O = 0; dividing by 1 there (not selecting 0) keeps a NaN row NaN, as the
      // reference's normalisation does (block_sparse_fa.py:255-257).
      const float r = O / (L > 0.f ? L : 1.f);
      p.o[b * p.so[0] + (int64_t)(h0 + gg) * p.so[1] + d] = f32_to16<DT>(r);
    } else {
      const int64_t row = ((int64_t)b * p.Hq + h0 + gg) * p.P + s;
      p.ws_o[row * D + d] = O;
      if (d == 0) {
        p.ws_ml[row * 2 + 0] = M;
        p.ws_ml[row * 2 + 1] = L;
      }
    }
  }
}

// Merge the P split partials of every (b, h) and write the output row.
template <int D, int DT>
__global__ void __launch_bounds__(D)
bsfa_decode_combine_kernel(const DecodeParams p) {
  const int64_t bh = blockIdx.x;
  const int b = (int)(bh / p.Hq);
  const int h = (int)(bh % p.Hq);
  const int d = threadIdx.x;
  const float* ml = p.ws_ml + bh * p.P * 2;
  const float* os = p.ws_o + bh * p.P * D;
  float M = -INFINITY;
  for (int sp = 0; sp < p.P; ++sp) M = fmaxf(M, ml[2 * sp]);
  const float Mu = (M == -INFINITY) ? 0.f : M;
  float L = 0.f, O = 0.f;
  for (int sp = 0; sp < p.P; ++sp) {
    const float f = __builtin_amdgcn_exp2f(ml[2 * sp] - Mu);
    L += ml[2 * sp + 1] * f;
    O += os[(int64_t)sp * D + d] * f;
  }
  const float r = O / (L > 0.f ? L : 1.f);  // empty rows: O = 0; NaN rows stay NaN
  p.o[b * p.so[0] + h * p.so[1] + d] = f32_to16<DT>(r);
}

template <int BS, int D, int MG, bool PAGED, int DT>
static hipError_t launch_decode_g(const DecodeParams& p, hipStream_t stream) {
  const int64_t grid = (int64_t)p.B * p.Hkv * p.P;
  hipLaunchKernelGGL((bsfa_decode_split_kernel<BS, D, MG, PAGED, DT>), dim3((unsigned)grid),
                     dim3(kDecodeWaves * kWave), 0, stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.P == 1) return err;
  hipLaunchKernelGGL((bsfa_decode_combine_kernel<D, DT>), dim3((unsigned)((int64_t)p.B * p.Hq)), dim3(D),
                     0, stream, p);
  return hipGetLastError();
}

template <int BS, int D, bool PAGED, int DT>
static hipError_t launch_decode_dt(const DecodeParams& p, hipStream_t stream) {
  if (p.G <= 1) return launch_decode_g<BS, D, 1, PAGED, DT>(p, stream);
  if (p.G <= 2) return launch_decode_g<BS, D, 2, PAGED, DT>(p, stream);
  if (p.G <= 4) return launch_decode_g<BS, D, 4, PAGED, DT>(p, stream);
  return launch_decode_g<BS, D, 8, PAGED, DT>(p, stream);
}

template <int BS, int D, bool PAGED = false>
static hipError_t launch_decode(const DecodeParams& p, int dtype, hipStream_t stream) {
  return dtype == kF16 ? launch_decode_dt<BS, D, PAGED, kF16>(p, stream)
                       : launch_decode_dt<BS, D, PAGED, kBf16>(p, stream);
}

}  // namespace tasft

using namespace tasft;

extern "C" size_t tasft_bsfa_decode_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                                    int64_t head_dim, int64_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || num_splits <= 0) return 0;
  return (size_t)(batch * num_q_heads * num_splits) * (size_t)(head_dim + 2) * sizeof(float);
}

static int decode_fwd(const void* q, const void* k_cache, const void* v_cache, void* out,
                      const uint8_t* block_mask, const int32_t* kv_lens, void* workspace,
                      size_t workspace_bytes, int64_t batch, int64_t num_q_heads,
                      int64_t num_kv_heads, int64_t kv_len_max, int64_t head_dim,
                      int64_t block_size, int64_t num_splits, const int64_t* q_strides,
                      const int64_t* k_strides, const int64_t* v_strides,
                      const int64_t* o_strides, const int64_t* mask_strides, float scale,
                      int dtype, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !block_mask || !workspace || !q_strides ||
      !k_strides || !v_strides || !o_strides || !mask_strides)
    return set_error(kErrInvalidArgument, "decode: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "decode: dtype must be bf16 (0) or fp16 (1), got %d", dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || kv_len_max <= 0 || num_splits <= 0)
    return set_error(kErrInvalidArgument, "decode: sizes must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "decode: num_q_heads must be a multiple of num_kv_heads");
  const int64_t G = num_q_heads / num_kv_heads;
  if (G > kDecodeMaxG)
    return set_error(kErrUnsupported, "decode: at most %d query heads per KV head, got %lld",
                     kDecodeMaxG, (long long)G);
  if (head_dim != 64 && head_dim != 128)
    return set_error(kErrUnsupported, "decode: head_dim must be 64 or 128, got %lld",
                     (long long)head_dim);
  if (block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(kErrUnsupported, "decode: block_size must be 32, 64 or 128, got %lld",
                     (long long)block_size);
  const int64_t nb = (kv_len_max + block_size - 1) / block_size;
  if ((nb + num_splits - 1) / num_splits > kDecodeMaxRange)
    return set_error(kErrInvalidArgument,
                     "decode: num_splits must be >= ceil(num_blocks / %d) (got %lld for %lld blocks)",
                     kDecodeMaxRange, (long long)num_splits, (long long)nb);
  const size_t need = tasft_bsfa_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
  if (workspace_bytes < need)
    return set_error(kErrWorkspace, "decode: workspace too small: need %zu bytes, got %zu", need,
                     workspace_bytes);
  if (!strides_nonneg(q_strides, 4) || !strides_nonneg(k_strides, 4) ||
      !strides_nonneg(v_strides, 4) || !strides_nonneg(o_strides, 4) ||
      !strides_nonneg(mask_strides, 4))
    return set_error(kErrInvalidArgument, "decode: strides must be non-negative");
  if (q_strides[3] != 1 || k_strides[3] != 1 || v_strides[3] != 1 || o_strides[3] != 1)
    return set_error(kErrInvalidArgument, "decode: head_dim must be the contiguous dimension");
  for (int j = 0; j < 3; ++j)
    if (k_strides[j] % 8 != 0 || v_strides[j] % 8 != 0)
      return set_error(kErrInvalidArgument, "decode: K/V strides must be multiples of 8 elements");
  if (q_strides[0] % 8 != 0 || q_strides[1] % 8 != 0)
    return set_error(kErrInvalidArgument, "decode: q strides must be multiples of 8 elements");
  if ((((uintptr_t)q) & 15u) || (((uintptr_t)k_cache) & 15u) || (((uintptr_t)v_cache) & 15u) ||
      (((uintptr_t)workspace) & 15u))
    return set_error(kErrInvalidArgument, "decode: q, K/V cache and workspace must be 16-byte aligned");
  if (batch * num_kv_heads * num_splits > 0x7fffffffLL || kv_len_max > 0x3fffffffLL)
    return set_error(kErrUnsupported, "decode: problem too large for one launch");

  DecodeParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k_cache;
  p.v = (const uint16_t*)v_cache;
  p.o = (uint16_t*)out;
  p.mask = block_mask;
  p.kv_lens = kv_lens;
  const size_t o_bytes = (size_t)(batch * num_q_heads * num_splits) * head_dim * sizeof(float);
  p.ws_o = (float*)workspace;
  p.ws_ml = (float*)((char*)workspace + o_bytes);
  p.sq[0] = q_strides[0];
  p.sq[1] = q_strides[1];
  p.so[0] = o_strides[0];
  p.so[1] = o_strides[1];
  for (int j = 0; j < 3; ++j) {
    p.sk[j] = k_strides[j];
    p.sv[j] = v_strides[j];
  }
  p.sm[0] = mask_strides[0];
  p.sm[1] = mask_strides[1];
  p.sm[2] = mask_strides[3];
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)G;
  p.S_kv = (int)kv_len_max;
  p.NB = (int)nb;
  p.P = (int)num_splits;
  p.scale_log2 = scale * kLog2e;

  p.block_table = nullptr;
  p.bt_stride = 0;
  p.page_size = 0;
  p.num_pages = 0;
  p.mshift = 0;

  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  if (block_size == 64 && head_dim == 128) err = launch_decode<64, 128>(p, dtype, s);
  else if (block_size == 64 && head_dim == 64) err = launch_decode<64, 64>(p, dtype, s);
  else if (block_size == 32 && head_dim == 128) err = launch_decode<32, 128>(p, dtype, s);
  else if (block_size == 32 && head_dim == 64) err = launch_decode<32, 64>(p, dtype, s);
  else if (block_size == 128 && head_dim == 128) err = launch_decode<128, 128>(p, dtype, s);
  else err = launch_decode<128, 64>(p, dtype, s);
  if (err != hipSuccess)
    return set_error(kErrLaunch, "decode: launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" int tasft_bsfa_decode_fwd(const void* q, const void* k_cache, const void* v_cache,
                                     void* out, const uint8_t* block_mask, const int32_t* kv_lens,
                                     void* workspace, size_t workspace_bytes, int64_t batch,
                                     int64_t num_q_heads, int64_t num_kv_heads, int64_t kv_len_max,
                                     int64_t head_dim, int64_t block_size, int64_t num_splits,
                                     const int64_t* q_strides, const int64_t* k_strides,
                                     const int64_t* v_strides, const int64_t* o_strides,
                                     const int64_t* mask_strides, float scale, int dtype,
                                     void* stream) {
  return decode_fwd(q, k_cache, v_cache, out, block_mask, kv_lens, workspace, workspace_bytes,
                    batch, num_q_heads, num_kv_heads, kv_len_max, head_dim, block_size,
                    num_splits, q_strides, k_strides, v_strides, o_strides, mask_strides, scale,
                    dtype, stream);
}

// ---------------------------------------------------------------------------- no allocation
// Static device scratch for tasft_bsfa_decode_fwd_noalloc: the split partials (the
// workspace of tasft_bsfa_decode_fwd) of every call on a GPU live in this one array, which
// each GPU the library runs on holds until the process ends. Its device address is taken
// once per device with hipGetSymbolAddress (the name itself is a host-side stand-in).
constexpr size_t kDecodeScratchBytes = TASFT_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

constexpr int kMaxScratchDevices = 64;

// Device address of `scratch` on the current device (looked up on the first call there).
static int decode_scratch_ptr(void** out) {
  static std::mutex mu;
  static void* ptrs[kMaxScratchDevices] = {};
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return set_error(kErrLaunch, "decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(kErrUnsupported, "decode_noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return set_error(kErrLaunch, "decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(err));
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return kOk;
}

extern "C" int tasft_bsfa_decode_fwd_noalloc(
    const void* q, const void* k_cache, const void* v_cache, void* out, const uint8_t* block_mask,
    const int32_t* kv_lens, int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t kv_len_max, int64_t head_dim, int64_t block_size, int64_t num_splits,
    const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
    const int64_t* o_strides, const int64_t* mask_strides, float scale, int dtype, void* stream) {
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "decode_noalloc: dtype must be bf16 (0) or fp16 (1), got %d",
                     dtype);
  const size_t need = tasft_bsfa_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
  if (need > kDecodeScratchBytes)
    return set_error(kErrWorkspace,
                     "decode_noalloc: %lld splits of %lld x %lld heads need %zu bytes of partials, "
                     "more than the %zu-byte static scratch (use fewer splits, or "
                     "tasft_bsfa_decode_fwd with a workspace)",
                     (long long)num_splits, (long long)batch, (long long)num_q_heads, need,
                     kDecodeScratchBytes);
  void* ws = nullptr;
  const int rc = decode_scratch_ptr(&ws);
  if (rc != kOk) return rc;
  return decode_fwd(q, k_cache, v_cache, out, block_mask, kv_lens, ws, kDecodeScratchBytes, batch,
                    num_q_heads, num_kv_heads, kv_len_max, head_dim, block_size, num_splits,
                    q_strides, k_strides, v_strides, o_strides, mask_strides, scale, dtype,
                    stream);
}

extern "C" int tasft_bsfa_decode_paged_fwd(
    const void* q, const void* k_pages, const void* v_pages, void* out, const uint8_t* block_mask,
    const int32_t* block_table, const int32_t* kv_lens, void* workspace, size_t workspace_bytes,
    int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t kv_len_max,
    int64_t head_dim, int64_t block_size, int64_t page_size, int64_t num_pages,
    int64_t num_splits, const int64_t* q_strides, const int64_t* k_strides,
    const int64_t* v_strides, const int64_t* o_strides, const int64_t* mask_strides,
    int64_t block_table_stride, float scale, int dtype, void* stream) {
  if (!q || !k_pages || !v_pages || !out || !block_mask || !block_table || !kv_lens ||
      !workspace || !q_strides || !k_strides || !v_strides || !o_strides || !mask_strides)
    return set_error(kErrInvalidArgument, "decode_paged: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "decode_paged: dtype must be bf16 (0) or fp16 (1), got %d",
                     dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || kv_len_max <= 0 || num_splits <= 0 ||
      num_pages <= 0)
    return set_error(kErrInvalidArgument, "decode_paged: sizes must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument,
                     "decode_paged: num_q_heads must be a multiple of num_kv_heads");
  const int64_t G = num_q_heads / num_kv_heads;
  if (G > kDecodeMaxG)
    return set_error(kErrUnsupported, "decode_paged: at most %d query heads per KV head, got %lld",
                     kDecodeMaxG, (long long)G);
  if (head_dim != 64 && head_dim != 128)
    return set_error(kErrUnsupported, "decode_paged: head_dim must be 64 or 128, got %lld",
                     (long long)head_dim);
  if (block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(kErrUnsupported, "decode_paged: block_size must be 32, 64 or 128, got %lld",
                     (long long)block_size);
  if (page_size < 8 || page_size > 4096 || (page_size & (page_size - 1)) != 0)
    return set_error(kErrUnsupported,
                     "decode_paged: page_size must be a power of two in [8, 4096], got %lld",
                     (long long)page_size);
  // A block-128 mask runs on the block-64 kernel: each selected 128-key block is read as
  // its two 64-key halves (mask entry t >> 1 for half t), so the split counts 64-key blocks.
  const int64_t run_bs = block_size == 128 ? 64 : block_size;
  const int64_t nb = (kv_len_max + run_bs - 1) / run_bs;
  if ((nb + num_splits - 1) / num_splits > kDecodeMaxRange)
    return set_error(kErrInvalidArgument,
                     "decode_paged: num_splits must be >= ceil(num_blocks / %d) (got %lld for %lld blocks of %lld keys)",
                     kDecodeMaxRange, (long long)num_splits, (long long)nb, (long long)run_bs);
  const size_t need = tasft_bsfa_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits);
  if (workspace_bytes < need)
    return set_error(kErrWorkspace, "decode_paged: workspace too small: need %zu bytes, got %zu",
                     need, workspace_bytes);
  // q, out [B, Hq, 1, D]; K/V pools [pages, page_size, Hkv, D].
  if (!strides_nonneg(q_strides, 4) || !strides_nonneg(k_strides, 4) ||
      !strides_nonneg(v_strides, 4) || !strides_nonneg(o_strides, 4) ||
      !strides_nonneg(mask_strides, 4) || block_table_stride < 0)
    return set_error(kErrInvalidArgument, "decode_paged: strides must be non-negative");
  if (q_strides[3] != 1 || k_strides[3] != 1 || v_strides[3] != 1 || o_strides[3] != 1)
    return set_error(kErrInvalidArgument, "decode_paged: head_dim must be the contiguous dimension");
  for (int j = 0; j < 3; ++j)
    if (k_strides[j] % 8 != 0 || v_strides[j] % 8 != 0)
      return set_error(kErrInvalidArgument,
                       "decode_paged: K/V strides must be multiples of 8 elements");
  if (q_strides[0] % 8 != 0 || q_strides[1] % 8 != 0)
    return set_error(kErrInvalidArgument, "decode_paged: q strides must be multiples of 8 elements");
  if ((((uintptr_t)q) & 15u) || (((uintptr_t)k_pages) & 15u) || (((uintptr_t)v_pages) & 15u) ||
      (((uintptr_t)workspace) & 15u))
    return set_error(kErrInvalidArgument,
                     "decode_paged: q, K/V pools and workspace must be 16-byte aligned");
  if (batch * num_kv_heads * num_splits > 0x7fffffffLL || kv_len_max > 0x3fffffffLL ||
      page_size * k_strides[1] * 2 > 0x7fffffffLL || page_size * v_strides[1] * 2 > 0x7fffffffLL ||
      num_pages > 0x7fffffffLL)
    return set_error(kErrUnsupported, "decode_paged: problem too large for one launch");

  DecodeParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k_pages;
  p.v = (const uint16_t*)v_pages;
  p.o = (uint16_t*)out;
  p.mask = block_mask;
  p.kv_lens = kv_lens;
  const size_t o_bytes = (size_t)(batch * num_q_heads * num_splits) * head_dim * sizeof(float);
  p.ws_o = (float*)workspace;
  p.ws_ml = (float*)((char*)workspace + o_bytes);
  p.sq[0] = q_strides[0];
  p.sq[1] = q_strides[1];
  p.so[0] = o_strides[0];
  p.so[1] = o_strides[1];
  // (page, head, token) strides of the pools.
  p.sk[0] = k_strides[0];
  p.sk[1] = k_strides[2];
  p.sk[2] = k_strides[1];
  p.sv[0] = v_strides[0];
  p.sv[1] = v_strides[2];
  p.sv[2] = v_strides[1];
  p.sm[0] = mask_strides[0];
  p.sm[1] = mask_strides[1];
  p.sm[2] = mask_strides[3];
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)G;
  p.S_kv = (int)kv_len_max;
  p.NB = (int)nb;
  p.P = (int)num_splits;
  p.scale_log2 = scale * kLog2e;
  p.block_table = block_table;
  p.bt_stride = block_table_stride;
  p.page_size = (int)page_size;
  p.num_pages = (int)num_pages;
  p.mshift = block_size == 128 ? 1 : 0;

  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  if (run_bs == 64 && head_dim == 128) err = launch_decode<64, 128, true>(p, dtype, s);
  else if (run_bs == 64 && head_dim == 64) err = launch_decode<64, 64, true>(p, dtype, s);
  else if (block_size == 32 && head_dim == 128) err = launch_decode<32, 128, true>(p, dtype, s);
  else err = launch_decode<32, 64, true>(p, dtype, s);
  if (err != hipSuccess)
    return set_error(kErrLaunch, "decode_paged: launch failed: %s", hipGetErrorString(err));
  return kOk;
}
