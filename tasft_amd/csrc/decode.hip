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
// Data path. A workgroup owns (batch b, KV head kvh, split s). The split is a share of
// the selected blocks: the blocks selected by any of the G query heads of kvh are
// numbered in block order and split s takes entries [s*n/P, (s+1)*n/P), so the splits of
// a row do equal work (a 128-key block counts as its two 64-key halves). Its 4 waves take the
// blocks round-robin. Each selected KV block is read from HBM once per KV
// head, however many query heads chose it; all its K and V loads are issued together.
// QK^T and PV both run on v_mfma_f32_16x16x32_bf16 (_f16 for fp16 inputs) with the G <= 16
// query heads of the KV head as the 16 N columns: K is loaded from HBM straight into the
// A-operand layout, V arrives in LDS by DMA and is read transposed (ds_read_b64_tr_b16) as
// the A operand of PV, and each lane's scores, probabilities and output columns belong
// to one head, so the softmax needs no LDS exchange. With one split the workgroup writes
// the output row; with several, partial (max, sum, output) triples per (b, h, split) go to
// a caller-provided workspace and a second kernel merges them.
#include "common.h"

#include <mutex>

#include "../../include/tasft_amd.h"

namespace tasft {

constexpr int kDecodeMaxG = 16;   // query heads per KV head handled by one workgroup
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

// v_mfma_f32_16x16x32_{bf16,f16}: 8 elements per lane of A and B as raw words.
template <int DT>
__device__ __forceinline__ f32x4_t mfma32k(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 16-byte chunk position of chunk `cc` of V row `r` in a wave's LDS tile. The PV operand
// reads (ds_read_b64_tr_b16) of 32 lanes touch rows r0 .. r0+7 (D = 128) or r0 .. r0+7
// with two 128-byte rows per 256 bytes (D = 64), two chunks each; the XOR spreads those
// 16 chunks over all 64 banks.
template <int D>
__device__ __forceinline__ int swz_dv(int r, int cc) {
  return D == 128 ? (cc ^ ((r & 7) << 1)) : (cc ^ (((r >> 1) & 3) << 1));
}

// The rotate-swap helpers of a 16-lane group: max / sum over the four lanes l % 16 + 16 g.
__device__ __forceinline__ float quad16_max(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return pair_max32(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float quad16_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return pair_sum32(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

// Keys of one KV block (BS = 32 or 64; a 128-key block runs as its two halves through the
// mask index shift) are processed by one wave. QK^T and PV both run on
// v_mfma_f32_16x16x32 with the query heads of the KV head as the 16 N columns (columns
// >= G carry zero queries and zero probabilities), so a lane owns one head: its scores,
// probabilities, rescale factor and output columns stay in its registers, and P^T is
// directly the B operand of the PV product. Up to 16 heads run two waves per SIMD.
template <int BS, int D, bool PAGED, int DT>
__global__ void __launch_bounds__(kDecodeWaves * kWave, 2)
bsfa_decode_split_kernel(const DecodeParams p) {
  static_assert(BS == 32 || BS == 64, "32- or 64-key blocks");
  constexpr int NT = BS / 16;         // 16-key score tiles per block
  constexpr int NC = BS / 32;         // 32-key PV k-steps per block
  constexpr int KS = D / 32;          // 32-dim QK k-steps
  constexpr int DT16 = D / 16;        // 16-dim output tiles
  constexpr int ROWB = D * 2;         // bytes of one K/V row
  constexpr int VTILE = BS * ROWB;    // bytes of one block of V
  constexpr int RPU = 1024 / ROWB;    // V rows per 1 KB DMA unit
  constexpr int CPR = ROWB / 16;      // 16-byte chunks per row
  __shared__ __attribute__((aligned(1024))) uint8_t v_lds[kDecodeWaves][VTILE];  // per-wave V tile
  __shared__ uint16_t hb[kDecodeMaxRange];  // head bits per selected entry
  __shared__ int sel[kDecodeMaxRange];      // selected blocks
  __shared__ int wsum[kDecodeWaves];
  __shared__ float comb_ml[kDecodeWaves][kDecodeMaxG][2];
  static_assert(kDecodeMaxG * D * 4 <= VTILE, "merge buffer size");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop state
  const int hc = lane & 15;   // query head (MFMA column) of this lane
  const int g4 = lane >> 4;   // lane group: keys 4*g4.. of a score tile, k slots 8*g4..
  const int G = p.G;

  const int64_t item = blockIdx.x;
  const int s = (int)(item % p.P);
  const int64_t bk = item / p.P;
  const int b = (int)(bk / p.Hkv);
  const int kvh = (int)(bk % p.Hkv);
  const int h0 = kvh * G;

  const int kv_len = p.kv_lens ? min(max(p.kv_lens[b], 0), p.S_kv) : p.S_kv;
  const int nb_valid = (kv_len + BS - 1) / BS;

  // Mask bits of key block t for the group's heads.
  const uint8_t* mbase = p.mask + b * p.sm[0] + (int64_t)h0 * p.sm[1];
  auto head_bits = [&](int t) -> uint32_t {
    uint32_t bitsv = 0;
    for (int gg = 0; gg < G; ++gg)
      if (mbase[(int64_t)gg * p.sm[1] + (int64_t)(t >> p.mshift) * p.sm[2]]) bitsv |= 1u << gg;
    return bitsv;
  };
  // Q^T as the B operand: lane (hc, g4) holds head h0+hc, head dims 32 ks + 8 g4 .. +7.
  u32x4_t qf[KS];
  {
    const bool hv = hc < G;
    const uint16_t* qrow = p.q + b * p.sq[0] + (int64_t)(h0 + (hv ? hc : 0)) * p.sq[1];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4_t val = {0u, 0u, 0u, 0u};
      if (hv) val = *(const u32x4_t*)(qrow + ks * 32 + g4 * 8);
      qf[ks] = val;
    }
  }

  const uint16_t* kbase = PAGED ? p.k + kvh * p.sk[1] : p.k + b * p.sk[0] + kvh * p.sk[1];
  const uint16_t* vbase = PAGED ? p.v + kvh * p.sv[1] : p.v + b * p.sv[0] + kvh * p.sv[1];
  const int ks2 = (int)p.sk[2], vs2 = (int)p.sv[2];  // row strides (elements)

  float m_run = -INFINITY, l_run = 0.f;  // this lane's head (equal over its four lane groups)
  f32x4_t oacc[DT16];                    // O^T tile dt: head hc, dims 16 dt + 4 g4 + j
#pragma unroll
  for (int dt = 0; dt < DT16; ++dt) oacc[dt] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  // K as the A operand: lane (hc, g4) loads key row 16 t + hc, dims 32 ks + 8 g4 .. +7.
  const int k_voff = (hc * ks2 + g4 * 8) * 2;
  // V DMA: lane l of unit u fetches the 16-byte chunk that the swizzle places at byte
  // u*1024 + 16*l of the tile, i.e. row u*RPU + l/CPR, position l%CPR. The whole offset
  // stays in the range-checked per-lane offset, so rows past kv_len read as zeros.
  auto v_src_off = [&](int u) {
    const int row = u * RPU + lane / CPR;
    return row * vs2 * 2 + swz_dv<D>(row, lane % CPR) * 16;
  };
  // V^T operand reads: lane (t = hc, g4) of a 16-lane group addresses row r0 + t/4 and the
  // 8 bytes of dims 16 dt + 4 (t%4) .. +3 (ds_read_b64_tr_b16 then hands lane t rows
  // r0 .. r0+3 of dim 16 dt + t).
  auto v_tr = [&](int r0, int dt) {
    const int row = r0 + (hc >> 2);
    const int d0 = dt * 16 + 4 * (hc & 3);
    return ds_read_tr16_b64((const void*)(v_lds[wave] + row * ROWB + swz_dv<D>(row, d0 >> 3) * 16 + (d0 & 7) * 2));
  };

  // Selected blocks of the split, compacted once, then taken round-robin by the waves.
  // Balanced splits: the blocks selected by any head of the group are numbered over the
  // whole row in block order, and split s takes entries [s*n/P, (s+1)*n/P). With one split
  // the count pass is skipped.
  constexpr int NTH = kDecodeWaves * kWave;
  int start = 0, end = 0x7fffffff;
  if (p.P > 1) {
    int cnt = 0;
    for (int t = tid; t < nb_valid; t += NTH) cnt += head_bits(t) != 0u ? 1 : 0;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) cnt += __shfl_xor(cnt, off, kWave);
    if (lane == 0) wsum[wave] = cnt;
    __syncthreads();
    const int n_all = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    start = (int)(((int64_t)s * n_all) / p.P);
    end = (int)(((int64_t)(s + 1) * n_all) / p.P);
    __syncthreads();  // wsum is rewritten below
  }
  int base = 0;
  for (int c0 = 0; c0 < nb_valid && base < end; c0 += NTH) {
    const int t = c0 + tid;
    const uint32_t bv = t < nb_valid ? head_bits(t) : 0u;
    const uint64_t bal = __ballot(bv != 0u);
    if (lane == 0) wsum[wave] = __popcll(bal);
    __syncthreads();
    int pos = base + __popcll(bal & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) pos += wsum[w];
    if (bv != 0u && pos >= start && pos < end) {
      sel[pos - start] = t;
      hb[pos - start] = (uint16_t)bv;
    }
    base += (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    __syncthreads();
  }
  const int nsel = __builtin_amdgcn_readfirstlane(min(end, base) - start);
  constexpr int NKL = NT * KS;  // K load instructions per block
  u32x4_t ka[NT][KS];
  // Paged cache: lane j < npg of `pgv` holds the page of the block's j-th page-sized piece
  // (one block ahead of use, so its load is covered by the fixed V wait).
  const int ps = p.page_size;
  const int npg = ps >= BS ? 1 : BS / ps;
  auto load_pg = [&](int kb) -> int {
    const int first = (kb * BS) / ps;
    // Only pages that hold a token below kv_len are read (later entries may not exist).
    const int jmax = (kv_len - 1 - kb * BS + (kb * BS) % ps) / ps;
    const int id = p.block_table[(int64_t)b * p.bt_stride + first + min(lane < npg ? lane : 0, jmax)];
    return min(max(id, 0), p.num_pages - 1);
  };
  auto load_k = [&](int kb, int pgv) {
    const int key0 = kb * BS;
    if constexpr (PAGED) {
      const int off0 = key0 % ps;
      if (ps >= 16) {
        // Every 16-key tile lies in one page (pages are powers of two >= 16, tiles start at
        // multiples of 16): one buffer resource per tile at a scalar page base, the per-lane
        // offsets of the contiguous path, and rows past kv_len read as zeros (masked).
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int row0 = off0 + t * 16;
          const int page = __builtin_amdgcn_readlane(pgv, row0 / ps);
          const int rows = min(16, kv_len - key0 - t * 16);
          const __amdgpu_buffer_rsrc_t kr = decode_rsrc(
              kbase + (int64_t)page * p.sk[0] + (int64_t)(row0 % ps) * ks2, (int64_t)max(rows, 0) * ks2 * 2);
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) ka[t][ks] = buf_load16(kr, k_voff + ks * 64, 0);
        }
      } else {
        const int last = kv_len - 1 - key0;  // rows past it read row kv_len-1 (masked)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int row = min(t * 16 + hc, last) + off0;
          const int page = __shfl(pgv, row / ps, kWave);
          const uint16_t* src = kbase + (int64_t)page * p.sk[0] + (int64_t)(row % ps) * ks2 + g4 * 8;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) ka[t][ks] = *(const u32x4_t*)(src + ks * 32);
        }
      }
    } else {
      const __amdgpu_buffer_rsrc_t kr = decode_rsrc(kbase + (int64_t)key0 * ks2, (int64_t)BS * ks2 * 2);
      if (key0 + BS <= kv_len) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) ka[t][ks] = buf_load16(kr, k_voff + ks * 64, t * 16 * ks2 * 2);
      } else {
        // Partial last block: K rows past kv_len are replaced by row kv_len-1; their
        // scores are masked to -inf.
        const int last = kv_len - 1 - key0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int row = min(t * 16 + hc, last);
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) ka[t][ks] = buf_load16(kr, (row * ks2 + g4 * 8) * 2 + ks * 64, 0);
        }
      }
    }
  };
  auto dma_v = [&](int kb, int pgv) {
    const int key0 = kb * BS;
    if constexpr (PAGED) {
      const int off0 = key0 % ps;
#pragma unroll
      for (int u = 0; u < VTILE / 1024; ++u) {
        // Unit u covers rows u*RPU .. +RPU-1 of the block, inside one page (ps % RPU == 0).
        const int row = u * RPU + off0;
        const int page = __builtin_amdgcn_readlane(pgv, row / ps);
        const int rows = min(RPU, kv_len - key0 - u * RPU);
        const __amdgpu_buffer_rsrc_t vr = decode_rsrc(
            vbase + (int64_t)page * p.sv[0] + (int64_t)(row % ps) * vs2, (int64_t)max(rows, 0) * vs2 * 2);
        dma16(vr, v_lds[wave] + u * 1024, v_src_off(u) - u * RPU * vs2 * 2);
      }
    } else {
      // The resource ends at row kv_len-1, so rows past kv_len arrive as zeros.
      const __amdgpu_buffer_rsrc_t vr =
          decode_rsrc(vbase + (int64_t)key0 * vs2, (int64_t)min(BS, kv_len - key0) * vs2 * 2);
#pragma unroll
      for (int u = 0; u < VTILE / 1024; ++u) dma16(vr, v_lds[wave] + u * 1024, v_src_off(u));
    }
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
    const bool head_on = hc < G && ((hsel >> hc) & 1u);
    // S^T = K Q^T: rows = keys, columns = heads.
    f32x4_t sacc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      sacc[t] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc[t] = mfma32k<DT>(ka[t][ks], qf[ks], sacc[t]);
    }
    // The next block of this wave: its K loads go out now (the K registers are free).
    const int en = e + kDecodeWaves;
    const bool more = en < nsel;
    const int tn = more ? __builtin_amdgcn_readfirstlane((int)sel[en]) : 0;
    int pg_nn = 0;
    if constexpr (PAGED) {
      // Pages of the block after the next, issued before the next block's K loads so the
      // fixed V wait below also covers them.
      const int enn = en + kDecodeWaves;
      pg_nn = load_pg(enn < nsel ? __builtin_amdgcn_readfirstlane((int)sel[enn]) : kb);
    }
    if (more) load_k(tn, pg_n);
    // Element j of tile t holds key 16 t + 4 g4 + j of head hc.
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = key0 + t * 16 + 4 * g4 + j;
        const float x = (head_on && key < kv_len) ? sacc[t][j] * p.scale_log2 : -INFINITY;
        sacc[t][j] = x;
        mx = fmaxf(mx, x);
      }
    mx = quad16_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float ls = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e2 = __builtin_amdgcn_exp2f(sacc[t][j] - m_use);
        sacc[t][j] = e2;
        ls += e2;
      }
    l_run = l_run * alpha + ls;
    m_run = m_new;
    // P^T as the B operand of k-step c: k slot 8 g4 + j holds key 32 c + 4 g4 + j (j < 4,
    // tile 2c) or 32 c + 16 + 4 g4 + j - 4 (tile 2c + 1), the order of the V^T reads below.
    u32x4_t pb[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
      pb[c] = (u32x4_t){pack16x2<DT>(sacc[2 * c][0], sacc[2 * c][1]), pack16x2<DT>(sacc[2 * c][2], sacc[2 * c][3]),
                        pack16x2<DT>(sacc[2 * c + 1][0], sacc[2 * c + 1][1]),
                        pack16x2<DT>(sacc[2 * c + 1][2], sacc[2 * c + 1][3])};
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) oacc[dt] *= alpha;
    // The V tile is private to this wave: wait for this block's V DMA (the next block's K
    // loads, issued after it, may still be in flight).
    if (more) __builtin_amdgcn_s_waitcnt(vmcnt_imm(NKL));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O^T += V^T P^T.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int r0 = 32 * c + 4 * g4;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) {
        const u32x2_t lo = v_tr(r0, dt), hi = v_tr(r0 + 16, dt);
        const u32x4_t a = {lo[0], lo[1], hi[0], hi[1]};
        oacc[dt] = mfma32k<DT>(a, pb[c], oacc[dt]);
      }
    }
    if (more) {
      // The DMA writes the V tile through the memory path: every LDS read of it must have
      // returned first.
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      dma_v(tn, pg_n);
    }
    pg_n = pg_nn;
    e = en;
  }

  // Merge the four waves: each wave's (m, l) per head and its output columns (into its
  // own V tile).
  __builtin_amdgcn_s_waitcnt(0x0f70);  // no V DMA may still target the tile
  const float l_tot = quad16_sum(l_run);
  if (g4 == 0 && hc < G) {
    comb_ml[wave][hc][0] = m_run;
    comb_ml[wave][hc][1] = l_tot;
  }
  if (hc < G) {
    float* mo = (float*)v_lds[wave];
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt)
      *(f32x4_t*)(mo + hc * D + dt * 16 + 4 * g4) = oacc[dt];
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += NTH) {
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

template <int BS, int D, bool PAGED, int DT>
static hipError_t launch_decode_dt(const DecodeParams& p, hipStream_t stream) {
  const int64_t grid = (int64_t)p.B * p.Hkv * p.P;
  hipLaunchKernelGGL((bsfa_decode_split_kernel<BS, D, PAGED, DT>), dim3((unsigned)grid),
                     dim3(kDecodeWaves * kWave), 0, stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.P == 1) return err;
  hipLaunchKernelGGL((bsfa_decode_combine_kernel<D, DT>), dim3((unsigned)((int64_t)p.B * p.Hq)), dim3(D),
                     0, stream, p);
  return hipGetLastError();
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
  // A block-128 mask runs on the block-64 kernel: each selected 128-key block is read as
  // its two 64-key halves (mask entry t >> 1 for half t), so the split counts 64-key blocks.
  const int64_t run_bs = block_size == 128 ? 64 : block_size;
  const int64_t nb = (kv_len_max + run_bs - 1) / run_bs;
  if ((nb + num_splits - 1) / num_splits > kDecodeMaxRange)
    return set_error(kErrInvalidArgument,
                     "decode: num_splits must be >= ceil(num_blocks / %d) (got %lld for %lld blocks of %lld keys)",
                     kDecodeMaxRange, (long long)num_splits, (long long)nb, (long long)run_bs);
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
  p.mshift = block_size == 128 ? 1 : 0;

  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  if (run_bs == 64 && head_dim == 128) err = launch_decode<64, 128>(p, dtype, s);
  else if (run_bs == 64 && head_dim == 64) err = launch_decode<64, 64>(p, dtype, s);
  else if (run_bs == 32 && head_dim == 128) err = launch_decode<32, 128>(p, dtype, s);
  else err = launch_decode<32, 64>(p, dtype, s);
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
