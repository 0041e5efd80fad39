// Causal GQA block-sparse flash-attention prefill for gfx950.
//
// Semantics follow the reference Triton kernel (tasft/kernels/block_sparse_fa.py:108-269)
// and its host preparation (:493-514):
//   * one query block of BS rows attends to the key blocks whose mask byte is non-zero;
//     with causal=1 the mask is AND-ed with the block lower triangle and, inside the
//     diagonal block, key > query is excluded;
//   * scores are fp32 (bf16 or fp16 MFMA, fp32 accumulate) times `scale`; online softmax in
//     fp32; P is rounded to the input type before the PV product (:252); l stays fp32;
//   * rows with no active key output 0 (:257-258); rows >= S are never stored (:268-269).
//
// GQA is native: query head h reads key/value head h / (Hq / Hkv) in place, so K/V are
// never expanded (the reference callers repeat_interleave them first,
// tasft/modules/tasft_attention.py:725-729).
//
// Mapping onto CDNA4. A workgroup owns one (batch, query head, query block) and has
// BS/32 waves; wave w owns 32 query rows. Each key block is computed as
// S^T = K . Q^T with v_mfma_f32_32x32x16_bf16 (_f16 for fp16 inputs), so a lane owns one query column of S^T:
// its running max and sum live in that lane (plus the lane 32 away), and the P^T
// accumulator registers feed the PV product O^T = V^T . P^T directly as the B operand
// with no shuffle. K (row major) and V^T (transposed while staging) go through LDS
// rows padded so the MFMA operand reads are bank-conflict free on the 64-bank LDS.
#include <algorithm>
#include <type_traits>

#include "common.h"


#include "../../include/tasft_amd.h"

namespace tasft {

struct PrefillParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  const uint8_t* mask;
  int64_t sq[3], sk[3], sv[3], so[3];  // element strides of dims (b, h, s); d stride is 1
  int64_t sm[4];                       // byte strides of the mask dims (b, h, qb, kb)
  int B, Hq, Hkv, G, S, NB;
  float scale_log2;  // softmax scale * log2(e)
  int causal;
  int small_spans;   // S * row bytes of K and V below 2^31: 32-bit DMA address math
  int* queue;        // per-partition ticket counters of the persistent launch, or null
  int parts;         // work partitions: 8 (one per XCD) or 1
  int wg_per_part;   // persistent workgroups per partition
  // Packed variable-length batch: sequence b holds tokens cu_seqlens[b] .. cu_seqlens[b+1]-1
  // of dimension s (the b strides are 0), S is the longest length and NB its block count.
  // Null for a dense [B, H, S, D] launch.
  const int* cu_seqlens;
  // Mask index shift: 64-token query block qb and key block kb read mask entry
  // (qb >> mshift, kb >> mshift). 1 runs a block-128 mask on the block-64 kernels (a
  // 128-token block is active iff each of its 64-token quarters is); 0 otherwise.
  int mshift;
};

// Static order of the (batch, query head, query block) work items. gfx950 dispatches
// workgroup i to XCD i % 8; each XCD walks the KV groups congruent to it modulo 8 one at
// a time (all query heads and query blocks of the group, longest causal rows first) so
// the group's K/V stays in that XCD's L2. With a number of KV groups that is not a
// multiple of 8 the order is group-major.
struct PrefillItem {
  int b, kvh, h, qb;
};

__device__ __forceinline__ PrefillItem prefill_item(const PrefillParams& p, int64_t idx64) {
  // 32-bit arithmetic: the host rejects B * Hq * NB >= 2^31.
  const uint32_t idx = (uint32_t)idx64;
  const uint32_t groups = (uint32_t)(p.B * p.Hkv);
  const uint32_t per_group = (uint32_t)(p.G * p.NB);
  uint32_t grp, r;
  if ((groups & 7) == 0) {
    const uint32_t j = idx >> 3;
    grp = (idx & 7) + 8 * (j / per_group);
    r = j % per_group;
  } else {
    grp = idx / per_group;
    r = idx % per_group;
  }
  const int qslot = (int)(r / (uint32_t)p.G);
  PrefillItem it;
  it.qb = p.causal ? (p.NB - 1 - qslot) : qslot;
  it.b = (int)(grp / (uint32_t)p.Hkv);
  it.kvh = (int)(grp % (uint32_t)p.Hkv);
  it.h = it.kvh * p.G + (int)(r % (uint32_t)p.G);
  return it;
}

// Token span of batch entry b: the whole sequence dimension (dense launch), or sequence b
// of a packed batch (its first token and length, clamped to [0, S]).
struct SeqSpan {
  int S, NB;
  int64_t tok0;
};

template <int BS>
__device__ __forceinline__ SeqSpan seq_span(const PrefillParams& p, int b) {
  if (!p.cu_seqlens) return {p.S, p.NB, 0};
  const int t0 = p.cu_seqlens[b];
  int len = p.cu_seqlens[b + 1] - t0;
  len = len < 0 ? 0 : (len > p.S ? p.S : len);
  return {len, (len + BS - 1) / BS, (int64_t)t0};
}

// Persistent launch (block size 64). Rows differ widely in cost (a gate can light whole
// rows), and a grid of one workgroup per row leaves CU slots idle while heavy and light
// rows are dispatched side by side. Instead, two workgroups per CU stay resident and
// pull rows from a ticket counter per partition (one partition per XCD: item
// x + 8j belongs to XCD x, so the static group-major order and its L2 locality are
// kept). The counters live in the caller's workspace and are zeroed by
// bsfa_queue_reset_kernel on the same stream before every launch.
constexpr int kQueueSlots = 8;

__global__ void bsfa_queue_reset_kernel(int* queue) {
  if (threadIdx.x < kQueueSlots) queue[threadIdx.x] = 0;
}

template <int BS, int D, int DT>
__global__ void __launch_bounds__(BS / 32 * kWave)
bsfa_prefill_kernel(const PrefillParams p) {
  constexpr int WAVES = BS / 32;
  constexpr int THREADS = WAVES * kWave;
  constexpr int KSTEPS = D / 16;   // MFMA k-steps over the head dim
  constexpr int KTILES = BS / 32;  // 32-key tiles per key block
  constexpr int DTILES = D / 32;   // 32-row head-dim tiles of O^T
  constexpr int KST = D + 8;       // LDS row stride of K (16-bit elements)
  constexpr int VST = BS + 4;      // LDS row stride of V^T (16-bit elements)

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[BS * KST];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VST];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;

  const PrefillItem item = prefill_item(p, (int64_t)blockIdx.x);
  const int qb = item.qb, b = item.b, kvh = item.kvh, h = item.h;
  // Varlen launch: items past the last query block of a shorter sequence have no work.
  const SeqSpan span = seq_span<BS>(p, b);
  if (qb >= span.NB) return;
  const int S = span.S, NB = span.NB;


  const uint16_t* qbase = p.q + b * p.sq[0] + span.tok0 * p.sq[2] + h * p.sq[1];
  const uint16_t* kbase = p.k + b * p.sk[0] + span.tok0 * p.sk[2] + kvh * p.sk[1];
  const uint16_t* vbase = p.v + b * p.sv[0] + span.tok0 * p.sv[2] + kvh * p.sv[1];
  uint16_t* obase = p.o + b * p.so[0] + span.tok0 * p.so[2] + h * p.so[1];
  const uint8_t* mrow = p.mask + b * p.sm[0] + h * p.sm[1] + (int64_t)(qb >> p.mshift) * p.sm[2];

  // Q^T as the B operand: lane (col, half) holds query row `qrow`, head dims
  // ks*16 + half*8 .. +7 for every k-step.
  const int qrow = qb * BS + wave * 32 + col;
  const bool qvalid = qrow < S;
  u32x4_t qf[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    u32x4_t val = {0u, 0u, 0u, 0u};
    if (qvalid) val = *(const u32x4_t*)(qbase + (int64_t)qrow * p.sq[2] + ks * 16 + half * 8);
    qf[ks] = val;
  }

  f32x16_t oacc[DTILES];
#pragma unroll
  for (int dt = 0; dt < DTILES; ++dt) oacc[dt] = (f32x16_t){};
  float m_run = -INFINITY;  // running max (log2 domain), identical in lanes l and l^32
  float l_run = 0.f;        // this lane's share of the running denominator

  const int kb_end = p.causal ? qb + 1 : NB;
  for (int chunk = 0; chunk < kb_end; chunk += kWave) {
    // Every wave reads the same 64 mask bytes, so all waves walk the same key blocks.
    const int kbl = chunk + lane;
    const bool act = (kbl < kb_end) && (mrow[(int64_t)(kbl >> p.mshift) * p.sm[3]] != 0);
    uint64_t bits = __ballot(act);
    while (bits) {
      const int kb = chunk + __builtin_ctzll(bits);
      bits &= bits - 1;
      const int key0 = kb * BS;

      __syncthreads();  // previous block's LDS reads are complete
      // Stage K rows (16-byte chunks), zero-filling keys >= S.
#pragma unroll
      for (int c = tid; c < BS * D / 8; c += THREADS) {
        const int r = c / (D / 8);
        const int cc = c % (D / 8);
        u32x4_t val = {0u, 0u, 0u, 0u};
        if (key0 + r < S) val = *(const u32x4_t*)(kbase + (int64_t)(key0 + r) * p.sk[2] + cc * 8);
        *(u32x4_t*)(k_lds + r * KST + cc * 8) = val;
      }
      // Stage V transposed: a unit is 4 keys x 8 head dims, written as 8 rows of V^T.
#pragma unroll
      for (int u = tid; u < (BS / 4) * (D / 8); u += THREADS) {
        const int kq = u % (BS / 4);
        const int dc = u / (BS / 4);
        u32x4_t rows[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = key0 + kq * 4 + j;
          rows[j] = (u32x4_t){0u, 0u, 0u, 0u};
          if (key < S) rows[j] = *(const u32x4_t*)(vbase + (int64_t)key * p.sv[2] + dc * 8);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          uint32_t e[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            e[j] = (i & 1) ? (rows[j][i >> 1] >> 16) : (rows[j][i >> 1] & 0xffffu);
          const u32x2_t w = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
          *(u32x2_t*)(vt_lds + (dc * 8 + i) * VST + kq * 4) = w;
        }
      }
      __syncthreads();

      // S^T tiles: rows = keys t*32 + ..., cols = this wave's 32 queries.
      f32x16_t s[KTILES];
#pragma unroll
      for (int t = 0; t < KTILES; ++t) {
        s[t] = (f32x16_t){};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const u32x4_t a = *(const u32x4_t*)(k_lds + (t * 32 + col) * KST + ks * 16 + half * 8);
          s[t] = mfma16<DT>(a, qf[ks], s[t]);
        }
      }

      // Register r of tile t holds key t*32 + 8*(r/4) + 4*half + r%4 for query `qrow`.
      const bool need_mask = (p.causal && kb == qb) || (key0 + BS > S);
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < KTILES; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[t][r] * p.scale_log2;
          if (need_mask) {
            const int key = key0 + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (key >= S || (p.causal && key > qrow)) x = -INFINITY;
          }
          s[t][r] = x;
          mloc = fmaxf(mloc, x);
        }
      }
      mloc = fmaxf(mloc, xor32(mloc));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float lsum = 0.f;
#pragma unroll
      for (int t = 0; t < KTILES; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(s[t][r] - m_use);
          s[t][r] = e;
          lsum += e;
        }
      }
      l_run = l_run * alpha + lsum;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) oacc[dt] *= alpha;

      // P^T as the B operand of O^T = V^T P^T: k-step (t, pp) uses registers 8pp..8pp+7
      // of tile t, i.e. keys t*32 + 16pp + 8*(j/4) + 4*half + j%4 for slot j.
      u32x4_t pb[KTILES][2];
#pragma unroll
      for (int t = 0; t < KTILES; ++t) {
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const u32x4_t w = {pack16x2<DT>(s[t][8 * pp + 0], s[t][8 * pp + 1]),
                             pack16x2<DT>(s[t][8 * pp + 2], s[t][8 * pp + 3]),
                             pack16x2<DT>(s[t][8 * pp + 4], s[t][8 * pp + 5]),
                             pack16x2<DT>(s[t][8 * pp + 6], s[t][8 * pp + 7])};
          pb[t][pp] = w;
        }
      }
      // V^T as the A operand with the same key order: two 4-key runs per slot group.
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
#pragma unroll
        for (int t = 0; t < KTILES; ++t) {
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            const uint16_t* vp = vt_lds + (dt * 32 + col) * VST + t * 32 + pp * 16 + half * 4;
            const u32x2_t lo = *(const u32x2_t*)vp;
            const u32x2_t hi = *(const u32x2_t*)(vp + 8);
            const u32x4_t a = {lo[0], lo[1], hi[0], hi[1]};
            oacc[dt] = mfma16<DT>(a, pb[t][pp], oacc[dt]);
          }
        }
      }
    }
  }

  // Epilogue: combine the two half-lane denominators, normalise, store in the input type.
  const float l_tot = l_run + xor32(l_run);
  const float inv = 1.f / (l_tot > 0.f ? l_tot : 1.f);  // empty rows: O = 0; NaN rows stay NaN
  if (qvalid) {
    uint16_t* orow = obase + (int64_t)qrow * p.so[2];
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = dt * 32 + 8 * gq + 4 * half;
        const u32x2_t w = {pack16x2<DT>(oacc[dt][4 * gq + 0] * inv, oacc[dt][4 * gq + 1] * inv),
                           pack16x2<DT>(oacc[dt][4 * gq + 2] * inv, oacc[dt][4 * gq + 3] * inv)};
        *(u32x2_t*)(orow + d0) = w;
      }
    }
  }
}

template <int BS, int D, int DT>
static hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream) {
  const int64_t grid = (int64_t)p.NB * p.B * p.Hq;
  hipLaunchKernelGGL((bsfa_prefill_kernel<BS, D, DT>), dim3((unsigned)grid), dim3(BS / 32 * kWave), 0,
                     stream, p);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------------------
// Block size 64: the tuned kernel.
//
// Four waves per (batch, query head, query block): wave w owns query rows 32*(w&1)..+31
// and the key half 32*(w>>1)..+31 of every key block, so each wave issues 8 + D/16 MFMAs
// per block and two waves share a SIMD. The two key-half partial results of a row are
// merged once at the end. K and V of the next active block are copied HBM -> LDS by
// buffer_load_dwordx4 ... lds (no staging registers) into the other of two LDS stages
// while the current block is computed (one barrier per block), row-major with a 16-byte
// XOR swizzle (conflict-free without padding). V^T operands come from
// ds_read_b64_tr_b16, so V is never transposed by VALU. The softmax rescale is lazy: the running maximum used
// for exp2 is only moved when a new score exceeds it by more than kRescaleLog2 (so P
// stays <= 2^8); numerator and denominator share the same reference, so the normalised
// output is unchanged.
// ---------------------------------------------------------------------------------------
constexpr float kRescaleLog2 = 8.f;

// 16-byte chunk position of chunk `cc` of K row `r` in LDS.
template <int D>
__device__ __forceinline__ int swz_k(int r, int cc) {
  return cc ^ (D == 128 ? (r & 15) : ((r >> 1) & 7));
}
// Same for V rows. ds_read_b64_tr_b16 serves 32 lanes (256 bytes) per LDS cycle: 4 rows
// x 4 chunks, which this swizzle spreads over all 64 banks.
template <int D>
__device__ __forceinline__ int swz_v(int r, int cc) {
  return cc ^ (D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2));
}

// Next active key block of a mask row, scanning 64 mask bytes per ballot. Returns -1 at
// the end. All lanes of all waves see the same sequence.
__device__ __forceinline__ int next_active_block(const uint8_t* mrow, int64_t stride, int kb_end,
                                                 int lane, int& chunk, uint64_t& bits,
                                                 int mshift) {
  while (bits == 0) {
    chunk += kWave;
    if (chunk >= kb_end) return -1;
    const int kbl = chunk + lane;
    bits = __ballot(kbl < kb_end && mrow[(int64_t)(kbl >> mshift) * stride] != 0);
  }
  const int kb = chunk + __builtin_ctzll(bits);
  bits &= bits - 1;
  return kb;
}

// One 64 x D 16-bit tile in LDS, written by buffer_load_dwordx4 ... lds (DMA, no VGPRs).
// Unit u (1 KB, one instruction of one wave) covers bytes u*1024 .. +1023 of the tile;
// lane l of that instruction lands at byte u*1024 + 16*l, i.e. row (u*1024+16l)/ROWB,
// 16-byte position ((u*1024+16l)%ROWB)/16. The lane therefore loads the global chunk
// that the swizzle maps to that position (the XOR swizzles are involutions). The
// buffer resource starts at the tile's first row and ends after row S-1, so rows past
// the end of the sequence are out of range and land in LDS as zeros.
template <int D>
__device__ __forceinline__ void dma_tile(uint8_t* tile, __amdgpu_buffer_rsrc_t rsrc,
                                         const int* voff, int wave) {
  constexpr int UNITS_PER_WAVE = (64 * D * 2 / 1024) / 4;
#pragma unroll
  for (int i = 0; i < UNITS_PER_WAVE; ++i) {
    const int u = wave * UNITS_PER_WAVE + i;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (TASFT_LDS void*)(tile + u * 1024), 16, voff[i], 0,
                                             0, 0);
  }
}

// Raw buffer resource (stride 0) over `bytes` bytes starting at `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, n, 0x00020000);
}

template <int D, int DT>
__global__ void __launch_bounds__(256, 2)
bsfa_prefill_bs64_kernel(const PrefillParams p) {
  constexpr int BS = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DTILES = D / 32;
  constexpr int ROWB = D * 2;                        // bytes per K/V row in LDS
  constexpr int TILE = BS * ROWB;                    // one K or V tile
  constexpr int UNITS_PER_WAVE = (TILE / 1024) / 4;  // DMA instructions per wave per tile

  // Two stages (A, B) of K and V tiles, each its own LDS object so that reads of one
  // stage are not ordered behind DMA into the other.
  __shared__ __attribute__((aligned(1024))) uint8_t kA[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t vA[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t kB[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t vB[TILE];
  __shared__ float xch_ml[2][2][2][32];  // (m, l) by row half, key half
  __shared__ int next_slot;
  static_assert(DTILES * 16 * kWave * 4 == TILE, "merge buffer size");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar DMA addresses
  const int rh = wave & 1;   // row half
  const int kh = wave >> 1;  // key half
  const int col = lane & 31;
  const int half = lane >> 5;

  // Per-lane byte offsets (within a tile's rows) of this wave's DMA units.
  int kvoff[UNITS_PER_WAVE], vvoff[UNITS_PER_WAVE];
#pragma unroll
  for (int i = 0; i < UNITS_PER_WAVE; ++i) {
    const int byte = (wave * UNITS_PER_WAVE + i) * 1024 + lane * 16;
    const int row = byte / ROWB, pos = (byte % ROWB) / 16;
    kvoff[i] = (row * (int)p.sk[2] + swz_k<D>(row, pos) * 8) * 2;
    vvoff[i] = (row * (int)p.sv[2] + swz_v<D>(row, pos) * 8) * 2;
  }
  const int krow_l = kh * 32 + col;
  const int grp16 = lane >> 4, t16 = lane & 15;  // ds_read_tr group and lane in group
  const int tr_row = t16 >> 2;                   // source row offset within a 4-row run
  const int tr_cb = t16 & 3;                     // source 8-byte column block

  // Work distribution: one item per workgroup, or the persistent ticket loop.
  const bool persistent = p.queue != nullptr;
  const int part = persistent ? (int)(blockIdx.x % p.parts) : 0;
  const int64_t per_part = persistent ? (int64_t)p.B * p.Hq * p.NB / p.parts : 1;
  int64_t slot = persistent ? (int64_t)(blockIdx.x / p.parts) : 0;
  // A workgroup knows its next item one item ahead: the second is static (slot +
  // wg_per_part), later ones come from tickets. The next item's first 64 mask bytes are
  // loaded during this item, so its first K/V DMA starts without a mask round trip.
  int64_t slot_nx = persistent ? slot + p.wg_per_part : per_part;
  bool pre = false;   // mbyte holds the first 64 mask bytes of this item's row, item_nx its item
  uint8_t mbyte = 0;
  PrefillItem item_nx = {0, 0, 0, 0};
  while (slot < per_part) {
  const int64_t idx = !persistent ? (int64_t)blockIdx.x : (p.parts == 8 ? part + 8 * slot : slot);
  const PrefillItem item = pre ? item_nx : prefill_item(p, idx);
  const int qb = item.qb, b = item.b, kvh = item.kvh, h = item.h;
  // Varlen launch: items past the last query block of a shorter sequence have no work.
  const SeqSpan span = seq_span<BS>(p, b);
  if (qb >= span.NB) return;  // (never in a persistent launch, which is dense)
  const int S = span.S, NB = span.NB;


  const uint16_t* qbase = p.q + b * p.sq[0] + span.tok0 * p.sq[2] + h * p.sq[1];
  const uint16_t* kbase = p.k + b * p.sk[0] + span.tok0 * p.sk[2] + kvh * p.sk[1];
  const uint16_t* vbase = p.v + b * p.sv[0] + span.tok0 * p.sv[2] + kvh * p.sv[1];
  uint16_t* obase = p.o + b * p.so[0] + span.tok0 * p.so[2] + h * p.so[1];
  const uint8_t* mrow = p.mask + b * p.sm[0] + h * p.sm[1] + (int64_t)(qb >> p.mshift) * p.sm[2];

  const int qrow = qb * BS + rh * 32 + col;
  const bool qvalid = qrow < S;
  const int kb_end = p.causal ? qb + 1 : NB;
  // Blocks from here on need element masks: the causal diagonal (the last block of a
  // causal row, which is also the partial block if there is one) or the partial block.
  const int mask_from = p.causal ? qb : ((S % BS) != 0 ? NB - 1 : NB);
  // Loads go out in the order their results are needed, since waits are in issue order:
  // this row's mask bytes (unless the previous item fetched them) and Q; the first K/V
  // DMA follows once the mask bytes are in, and only then the next item's mask bytes and
  // the ticket of the item after the next, which the first wait also covers.
  uint8_t mb = mbyte;
  if (!pre && lane < kb_end) mb = mrow[(int64_t)(lane >> p.mshift) * p.sm[3]];
  u32x4_t qf[KSTEPS];
  {
    // Rows past the end read row S-1: per-row results, never stored.
    const uint16_t* qr = qbase + (int64_t)(qvalid ? qrow : S - 1) * p.sq[2] + half * 8;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[ks] = *(const u32x4_t*)(qr + ks * 16);
  }
  // Start the DMA of key block kb into one stage (rows >= S arrive as zeros). With
  // small spans the resource base and size take 32-bit scalar math only.
  const uint32_t krb = (uint32_t)p.sk[2] * 2u, vrb = (uint32_t)p.sv[2] * 2u;
  auto issue = [&](uint8_t* kt, uint8_t* vt, int kb) {
    if (p.small_spans) {
      const uint32_t key0 = (uint32_t)kb * BS, left = (uint32_t)S - key0;
      dma_tile<D>(kt, __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)kbase + key0 * krb),
                                                        (short)0, (int)(left * krb), 0x00020000),
                  kvoff, wave);
      dma_tile<D>(vt, __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)vbase + key0 * vrb),
                                                        (short)0, (int)(left * vrb), 0x00020000),
                  vvoff, wave);
    } else {
      const int key0 = kb * BS;
      const int64_t rows_left = (int64_t)(S - key0);
      dma_tile<D>(kt, tile_rsrc(kbase + (int64_t)key0 * p.sk[2], rows_left * p.sk[2] * 2), kvoff, wave);
      dma_tile<D>(vt, tile_rsrc(vbase + (int64_t)key0 * p.sv[2], rows_left * p.sv[2] * 2), vvoff, wave);
    }
  };

  f32x16_t oacc[DTILES];
#pragma unroll
  for (int dt = 0; dt < DTILES; ++dt) oacc[dt] = (f32x16_t){};
  float m_ref = -INFINITY;  // exp2 reference of this lane's query row (log2 domain)
  float l_run = 0.f;

  // One key block from stage (kt, vt): S^T MFMAs, online softmax, PV MFMAs.
  auto compute = [&](const uint8_t* kt, const uint8_t* vt, int kb) {
    // Every LDS operand of the block is requested before the first MFMA: the K fragments,
    // then (behind a scheduling fence) the V^T fragments, whose reads the S MFMAs cover.
    u32x4_t kf[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cc = ks * 2 + half;
      kf[ks] = *(const u32x4_t*)(kt + krow_l * ROWB + swz_k<D>(krow_l, cc) * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x2_t vlo[2][DTILES], vhi[2][DTILES];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const int kbase_k = kh * 32 + 16 * pp + 4 * (grp16 >> 1);  // first key of run 1
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const int d0 = dt * 32 + 16 * (grp16 & 1) + 4 * tr_cb;  // source column of this lane
        const int cc = d0 >> 3, sub = (d0 & 7) * 2;
        const int r1 = kbase_k + tr_row, r2 = r1 + 8;
        vlo[pp][dt] = ds_read_tr16_b64((const void*)(vt + r1 * ROWB + swz_v<D>(r1, cc) * 16 + sub));
        vhi[pp][dt] = ds_read_tr16_b64((const void*)(vt + r2 * ROWB + swz_v<D>(r2, cc) * 16 + sub));
      }
    }
    f32x16_t s = (f32x16_t){};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) s = mfma16<DT>(kf[ks], qf[ks], s);
    // Each S MFMA followed by two V^T reads.
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    const int key0 = kb * BS;
    // Causal diagonal block or partial last block: mask in one uniform branch.
    if (kb >= mask_from) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int key = key0 + kh * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
        s[rr] = (key >= S || (p.causal && key > qrow)) ? -INFINITY : s[rr];
      }
    }
    // Scores stay unscaled: scale > 0 commutes with max, and exp2 takes one FMA.
    float mraw = s[0];
#pragma unroll
    for (int rr = 1; rr < 16; ++rr) mraw = fmaxf(mraw, s[rr]);
    const float mloc = pair_max32(mraw) * p.scale_log2;
    // Lazy rescale: move the reference only when a score exceeds it by kRescaleLog2.
    const bool move = mloc > m_ref + kRescaleLog2;
    if (__ballot(move)) {
      // exp2(-inf) = 0 clears the (empty) accumulators on a row's first finite score.
      const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - mloc) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) oacc[dt] *= alpha;
      m_ref = move ? mloc : m_ref;
    }
    const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
    float lsum = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float e = __builtin_amdgcn_exp2f(fmaf(s[rr], p.scale_log2, -m_use));
      s[rr] = e;
      lsum += e;
    }
    l_run += lsum;
    // O^T += V^T P^T over this wave's 32 keys: two k-steps of 16 keys.
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const u32x4_t w = {pack16x2<DT>(s[8 * pp + 0], s[8 * pp + 1]),
                         pack16x2<DT>(s[8 * pp + 2], s[8 * pp + 3]),
                         pack16x2<DT>(s[8 * pp + 4], s[8 * pp + 5]),
                         pack16x2<DT>(s[8 * pp + 6], s[8 * pp + 7])};
      const u32x4_t pb = w;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const u32x4_t a = {vlo[pp][dt][0], vlo[pp][dt][1], vhi[pp][dt][0], vhi[pp][dt][1]};
        oacc[dt] = mfma16<DT>(a, pb, oacc[dt]);
      }
    }
  };

  int chunk = 0;
  uint64_t bits = __ballot(mb != 0);
  int kb = next_active_block(mrow, p.sm[3], kb_end, lane, chunk, bits, p.mshift);
  if (kb >= 0) issue(kA, vA, kb);
  mbyte = 0;
  pre = slot_nx < per_part;
  if (pre) {
    item_nx = prefill_item(p, p.parts == 8 ? part + 8 * slot_nx : slot_nx);
    const int kb_end_nx = p.causal ? item_nx.qb + 1 : p.NB;
    const uint8_t* mrow_nx =
        p.mask + item_nx.b * p.sm[0] + item_nx.h * p.sm[1] + (int64_t)(item_nx.qb >> p.mshift) * p.sm[2];
    if (lane < kb_end_nx) mbyte = mrow_nx[(int64_t)(lane >> p.mshift) * p.sm[3]];
  }
  // atomicInc (not atomicAdd, which the compiler rewrites into a wave-aggregated form that
  // waits for the result on the spot); the counter never reaches the wrap limit.
  int ticket = 0;
  if (persistent && tid == 0) ticket = (int)atomicInc((unsigned*)&p.queue[part], 0xffffffffu);
  // Unrolled by two so each stage is a fixed LDS object.
  while (kb >= 0) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's DMA of block kb landed
    __syncthreads();                      // every wave's DMA landed; stage B is free
    int kb_next = next_active_block(mrow, p.sm[3], kb_end, lane, chunk, bits, p.mshift);
    if (kb_next >= 0) issue(kB, vB, kb_next);
    compute(kA, vA, kb);
    kb = kb_next;
    if (kb < 0) break;
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    kb_next = next_active_block(mrow, p.sm[3], kb_end, lane, chunk, bits, p.mshift);
    if (kb_next >= 0) issue(kA, vA, kb_next);
    compute(kB, vB, kb);
    kb = kb_next;
  }

  // Merge the two key halves of each row. Each wave finalises half of the head dims (key
  // half 0 the first DTILES/2 tiles, key half 1 the rest) and hands its partner the other
  // half of its partial O^T and its (m, l), through stage A.
  constexpr int HT = DTILES / 2;
  const float l_tot = pair_sum32(l_run);
  __syncthreads();  // every wave is done with stage A
  float* xo = (float*)(rh == 0 ? kA : vA);  // 2 x HT tiles of 16 x 64 floats per row half
  auto send = [&](auto khc) {
    constexpr int KH = decltype(khc)::value;
    float* out = xo + KH * (HT * 16 * kWave);
#pragma unroll
    for (int j = 0; j < HT; ++j)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) out[(j * 16 + rr) * kWave + lane] = oacc[(1 - KH) * HT + j][rr];
    if (half == 0) {
      xch_ml[rh][KH][0][col] = m_ref;
      xch_ml[rh][KH][1][col] = l_tot;
    }
  };
  auto finish = [&](auto khc) {
    constexpr int KH = decltype(khc)::value;
    const float* in = xo + (1 - KH) * (HT * 16 * kWave);
    const float mp = xch_ml[rh][1 - KH][0][col], lp = xch_ml[rh][1 - KH][1][col];
    // The same expressions in both waves, in key-half order.
    const float m0 = KH == 0 ? m_ref : mp, m1 = KH == 0 ? mp : m_ref;
    const float l0 = KH == 0 ? l_tot : lp, l1 = KH == 0 ? lp : l_tot;
    const float M = fmaxf(m0, m1);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    const float f0 = __builtin_amdgcn_exp2f(m0 - Mu);  // 0 for an empty half
    const float f1 = __builtin_amdgcn_exp2f(m1 - Mu);
    const float L = l0 * f0 + l1 * f1;
    const float inv = 1.f / (L > 0.f ? L : 1.f);  // empty rows: O = 0; NaN rows stay NaN
    if (qvalid) {
      uint16_t* orow = obase + (int64_t)qrow * p.so[2];
#pragma unroll
      for (int j = 0; j < HT; ++j) {
        const int dt = KH * HT + j;
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          float o4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int rr = 4 * gq + e;
            const float mine = oacc[dt][rr], theirs = in[(j * 16 + rr) * kWave + lane];
            const float p0 = KH == 0 ? mine : theirs, p1 = KH == 0 ? theirs : mine;
            o4[e] = (p0 * f0 + p1 * f1) * inv;
          }
          const int d0 = dt * 32 + 8 * gq + 4 * half;
          const u32x2_t w = {pack16x2<DT>(o4[0], o4[1]), pack16x2<DT>(o4[2], o4[3])};
          *(u32x2_t*)(orow + d0) = w;
        }
      }
    }
  };
  if (kh == 0)
    send(std::integral_constant<int, 0>{});
  else
    send(std::integral_constant<int, 1>{});
  __syncthreads();
  if (kh == 0)
    finish(std::integral_constant<int, 0>{});
  else
    finish(std::integral_constant<int, 1>{});
  if (!persistent) break;
  if (tid == 0) next_slot = 2 * p.wg_per_part + ticket;
  __syncthreads();  // merge buffer, stages and next_slot are free for the next item
  slot = slot_nx;
  slot_nx = __builtin_amdgcn_readfirstlane(next_slot);
  }
}

// ---------------------------------------------------------------------------------------
// Block size 64, head dim 128: two waves per query block.
//
// Wave w owns query rows 32*w..+31 and all 64 keys of every active key block: 16 S MFMAs
// (two 32-key tiles) and 16 PV MFMAs per block, so a row needs no merge of partial
// results. Four such workgroups (32 KB of LDS each: one K tile and one V tile) share a CU,
// two waves per SIMD. Per block: the V DMA starts once every wave has read the previous
// V tile, and the next block's K DMA once every wave has read this K tile; PV waits for V
// only. The barriers carry no memory fence (a __syncthreads() fence would also wait for
// the DMA still in flight): each is preceded by the explicit wait it needs. Each DMA
// instruction moves 1 KB; one LDS base (M0) serves four of them
// through the instruction offset, which the hardware adds to both the global and the LDS
// address (the field holds 12 bits, so units four apart need their own base).
// Q and O pass through the V tile, which is free before the row's first V DMA and after
// its last PV: Q arrives by DMA in the K layout (whole 256-byte rows per request) and is
// read into the MFMA operand registers like K; O is written there per wave and stored as
// whole rows, four per instruction. Loading Q and storing O directly in the MFMA layouts
// touched 32 rows, 32 bytes each, per instruction (1 KB of data in 32 cache lines).
// ---------------------------------------------------------------------------------------
// Workgroup barrier without a memory fence. The caller waits (s_waitcnt) for what the
// barrier publishes; the memory clobber keeps the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// AUX: the DMA's cache policy bits (0: default; 2: non-temporal, for Q, which a row reads
// once, so that it does not push its KV group's K and V out of L2).
template <int D, int AUX = 0>
__device__ __forceinline__ void dma_tile_2w(uint8_t* tile, __amdgpu_buffer_rsrc_t rsrc,
                                            const int* voff, int wave) {
  static_assert(D == 128, "eight 1 KB units per wave and tile");
  TASFT_LDS void* b0 = (TASFT_LDS void*)(tile + wave * 8192);
  TASFT_LDS void* b1 = (TASFT_LDS void*)(tile + wave * 8192 + 4096);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b0, 16, voff[0], 0, 0, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b0, 16, voff[1], 0, 1024, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b0, 16, voff[2], 0, 2048, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b0, 16, voff[3], 0, 3072, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b1, 16, voff[4], 0, 0, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b1, 16, voff[5], 0, 1024, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b1, 16, voff[6], 0, 2048, AUX);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, b1, 16, voff[7], 0, 3072, AUX);
}

template <int D, int DT>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2, 2)))
bsfa_prefill_bs64_2w_kernel(const PrefillParams p) {
  constexpr int BS = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DTILES = D / 32;
  constexpr int ROWB = D * 2;
  constexpr int TILE = BS * ROWB;
  constexpr int UPW = (TILE / 1024) / 2;  // DMA units per wave and tile

  __shared__ __attribute__((aligned(1024))) uint8_t kS[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t vS[TILE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar DMA addresses
  const int col = lane & 31;
  const int half = lane >> 5;

  // Per-lane source offsets of this wave's DMA units (see dma_tile), less the instruction
  // offset that dma_tile_2w adds. Unit u starts at tile row 4u >= 4 (u & 3), so the
  // difference stays non-negative.
  int kvoff[UPW], vvoff[UPW];
#pragma unroll
  for (int i = 0; i < UPW; ++i) {
    const int byte = (wave * UPW + i) * 1024 + lane * 16;
    const int row = byte / ROWB, pos = (byte % ROWB) / 16;
    kvoff[i] = (row * (int)p.sk[2] + swz_k<D>(row, pos) * 8) * 2 - (i & 3) * 1024;
    vvoff[i] = (row * (int)p.sv[2] + swz_v<D>(row, pos) * 8) * 2 - (i & 3) * 1024;
  }
  const int grp16 = lane >> 4, t16 = lane & 15;  // ds_read_tr group and lane in group
  const int tr_row = t16 >> 2;                   // source row offset within a 4-row run
  const int tr_cb = t16 & 3;                     // source 8-byte column block
  const uint32_t krb = (uint32_t)p.sk[2] * 2u, vrb = (uint32_t)p.sv[2] * 2u;

  const PrefillItem item = prefill_item(p, (int64_t)blockIdx.x);
  const int qb = item.qb, b = item.b, kvh = item.kvh, h = item.h;
  // Varlen launch: items past the last query block of a shorter sequence have no work.
  const SeqSpan span = seq_span<BS>(p, b);
  if (qb >= span.NB) return;
  const int S = span.S, NB = span.NB;


  const uint16_t* qbase = p.q + b * p.sq[0] + span.tok0 * p.sq[2] + h * p.sq[1];
  const uint16_t* kbase = p.k + b * p.sk[0] + span.tok0 * p.sk[2] + kvh * p.sk[1];
  const uint16_t* vbase = p.v + b * p.sv[0] + span.tok0 * p.sv[2] + kvh * p.sv[1];
  uint16_t* obase = p.o + b * p.so[0] + span.tok0 * p.so[2] + h * p.so[1];
  const uint8_t* mrow = p.mask + b * p.sm[0] + h * p.sm[1] + (int64_t)(qb >> p.mshift) * p.sm[2];

  const int qrow = qb * BS + wave * 32 + col;
  const int kb_end = p.causal ? qb + 1 : NB;
  // Blocks from here on need element masks (causal diagonal or partial last block).
  const int mask_from = p.causal ? qb : ((S % BS) != 0 ? NB - 1 : NB);
  // Loads in the order their results are needed: mask bytes, Q, then the first K DMA.
  uint8_t mb = 0;
  if (lane < kb_end) mb = mrow[(int64_t)(lane >> p.mshift) * p.sm[3]];
  // The query block's rows go HBM->LDS by DMA into the V tile (unused until the first V
  // DMA), in the K tile's swizzled layout: each 1 KB unit is 4 whole rows, so every
  // request covers full cache lines. Rows past the end arrive as zeros (never stored).
  {
    int qvoff[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int byte = (wave * UPW + i) * 1024 + lane * 16;
      const int row = byte / ROWB, pos = (byte % ROWB) / 16;
      qvoff[i] = (row * (int)p.sq[2] + swz_k<D>(row, pos) * 8) * 2 - (i & 3) * 1024;
    }
    dma_tile_2w<D, 2>(vS, tile_rsrc(qbase + (int64_t)qb * BS * p.sq[2], (int64_t)(S - qb * BS) * p.sq[2] * 2),
                      qvoff, wave);
  }
  // Buffer resource of key block kb of K or V (rows >= S are out of range: zeros).
  auto block_rsrc = [&](const uint16_t* base, uint32_t rb, int64_t stride, int kb) {
    if (p.small_spans) {
      const uint32_t key0 = (uint32_t)kb * BS, left = (uint32_t)S - key0;
      return __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)base + key0 * rb), (short)0,
                                               (int)(left * rb), 0x00020000);
    }
    const int key0 = kb * BS;
    return tile_rsrc(base + (int64_t)key0 * stride, (int64_t)(S - key0) * stride * 2);
  };

  f32x16_t oacc[DTILES];
#pragma unroll
  for (int dt = 0; dt < DTILES; ++dt) oacc[dt] = (f32x16_t){};
  float m_ref = -INFINITY;  // exp2 reference of this lane's query row (log2 domain)
  float l_run = 0.f;

  int chunk = 0;
  uint64_t bits = __ballot(mb != 0);
  int kb = next_active_block(mrow, p.sm[3], kb_end, lane, chunk, bits, p.mshift);
  u32x4_t qf[KSTEPS];
  if (kb >= 0) {
    dma_tile_2w<D>(kS, block_rsrc(kbase, krb, p.sk[2], kb), kvoff, wave);
    __builtin_amdgcn_s_waitcnt(0x0f78);  // vmcnt(8): own share of Q landed, K in flight
  } else {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  }
  block_barrier();  // Q visible; the loop's first barrier orders these reads before V's DMA
  {
    const int r = wave * 32 + col;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qf[ks] = *(const u32x4_t*)(vS + r * ROWB + swz_k<D>(r, ks * 2 + half) * 16);
  }

  while (kb >= 0) {
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): own share of K(kb) landed
    block_barrier();                      // K(kb) visible; every wave is done with the V tile
    dma_tile_2w<D>(vS, block_rsrc(vbase, vrb, p.sv[2], kb), vvoff, wave);
    u32x4_t kf[2][KSTEPS];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int r = kt * 32 + col;
        kf[kt][ks] = *(const u32x4_t*)(kS + r * ROWB + swz_k<D>(r, ks * 2 + half) * 16);
      }
    f32x16_t s0 = (f32x16_t){}, s1 = (f32x16_t){};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      s0 = mfma16<DT>(kf[0][ks], qf[ks], s0);
      s1 = mfma16<DT>(kf[1][ks], qf[ks], s1);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's K reads returned
    block_barrier();                      // every wave has read K(kb): the K tile is free
    const int kb_next = next_active_block(mrow, p.sm[3], kb_end, lane, chunk, bits, p.mshift);
    // Always eight DMA units after V(kb) (the last block of a row loads its own K tile
    // again), so the V wait below is one fixed count.
    dma_tile_2w<D>(kS, block_rsrc(kbase, krb, p.sk[2], kb_next >= 0 ? kb_next : kb), kvoff, wave);
    if (kb >= mask_from) {
      // Register rr of tile t holds key kb*BS + 32t + 4*half + off(rr), off = 8*(rr/4) +
      // rr%4; a key is admissible iff it is <= min(qrow, S-1) (causal) or S-1, i.e. iff
      // 32t + off <= lim below: one compare per score.
      const int last = p.causal ? min(qrow, S - 1) : S - 1;
      const int lim = last - kb * BS - 4 * half;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int off = 8 * (rr >> 2) + (rr & 3);
        s0[rr] = off > lim ? -INFINITY : s0[rr];
        s1[rr] = off + 32 > lim ? -INFINITY : s1[rr];
      }
    }
    // Scores stay unscaled: scale > 0 commutes with max, and exp2 takes one FMA. Two
    // chains of three-input maxima.
    float ma = fmaxf(fmaxf(s0[0], s0[1]), s0[2]), mb = fmaxf(fmaxf(s1[0], s1[1]), s1[2]);
#pragma unroll
    for (int rr = 3; rr < 15; rr += 2) {
      ma = fmaxf(fmaxf(ma, s0[rr]), s0[rr + 1]);
      mb = fmaxf(fmaxf(mb, s1[rr]), s1[rr + 1]);
    }
    const float mraw = fmaxf(fmaxf(ma, s0[15]), fmaxf(mb, s1[15]));
    const float mloc = pair_max32(mraw) * p.scale_log2;
    const bool move = mloc > m_ref + kRescaleLog2;
    if (__ballot(move)) {
      // exp2(-inf) = 0 clears the (empty) accumulators on a row's first finite score.
      const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - mloc) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) oacc[dt] *= alpha;
      m_ref = move ? mloc : m_ref;
    }
    const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
    float lsum0 = 0.f, lsum1 = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float e0 = __builtin_amdgcn_exp2f(fmaf(s0[rr], p.scale_log2, -m_use));
      const float e1 = __builtin_amdgcn_exp2f(fmaf(s1[rr], p.scale_log2, -m_use));
      s0[rr] = e0;
      s1[rr] = e1;
      lsum0 += e0;
      lsum1 += e1;
    }
    l_run += lsum0 + lsum1;
    // P^T as the B operand of four 16-key k-steps: keys 16pp + 8*(j>>2) + 4*half + (j&3)
    // for element j, the same key order the V^T reads below use.
    u32x4_t pb[4];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const f32x16_t& sv = (pp < 2) ? s0 : s1;
      const int o = 8 * (pp & 1);
      const u32x4_t w = {pack16x2<DT>(sv[o + 0], sv[o + 1]), pack16x2<DT>(sv[o + 2], sv[o + 3]),
                         pack16x2<DT>(sv[o + 4], sv[o + 5]), pack16x2<DT>(sv[o + 6], sv[o + 7])};
      pb[pp] = w;
    }
    __builtin_amdgcn_s_waitcnt(0x0f78);  // vmcnt(8): own share of V(kb) landed, next K in flight
    block_barrier();                      // V(kb) visible
    u32x2_t vlo[4][DTILES], vhi[4][DTILES];
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const int kk = 16 * pp + 4 * (grp16 >> 1);  // first key of run 1
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const int d0 = dt * 32 + 16 * (grp16 & 1) + 4 * tr_cb;  // source column of this lane
        const int cc = d0 >> 3, sub = (d0 & 7) * 2;
        const int r1 = kk + tr_row, r2 = r1 + 8;
        vlo[pp][dt] = ds_read_tr16_b64((const void*)(vS + r1 * ROWB + swz_v<D>(r1, cc) * 16 + sub));
        vhi[pp][dt] = ds_read_tr16_b64((const void*)(vS + r2 * ROWB + swz_v<D>(r2, cc) * 16 + sub));
      }
    }
#pragma unroll
    for (int pp = 0; pp < 4; ++pp)
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        const u32x4_t a = {vlo[pp][dt][0], vlo[pp][dt][1], vhi[pp][dt][0], vhi[pp][dt][1]};
        oacc[dt] = mfma16<DT>(a, pb[pp], oacc[dt]);
      }
    kb = kb_next;
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // no DMA into this workgroup's LDS outlives it

  const float l_tot = pair_sum32(l_run);
  const float inv = 1.f / (l_tot > 0.f ? l_tot : 1.f);  // empty rows: O = 0; NaN rows stay NaN
  // The output through LDS: each wave writes its 32 rows into its own 8 KB of the V tile
  // (16-byte chunk c of row r at position c ^ (r & 15)), then stores whole 256-byte rows,
  // four rows per instruction.
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's V reads returned
  block_barrier();                      // every wave is done with the V tile
  uint8_t* ost = vS + wave * (32 * ROWB);
#pragma unroll
  for (int dt = 0; dt < DTILES; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d0 = dt * 32 + 8 * gq + 4 * half;
      const u32x2_t w = {pack16x2<DT>(oacc[dt][4 * gq + 0] * inv, oacc[dt][4 * gq + 1] * inv),
                         pack16x2<DT>(oacc[dt][4 * gq + 2] * inv, oacc[dt][4 * gq + 3] * inv)};
      *(u32x2_t*)(ost + col * ROWB + (((d0 >> 3) ^ (col & 15)) << 4) + (d0 & 7) * 2) = w;
    }
  constexpr int CPR = ROWB / 16;  // 16-byte chunks per row
  const int row0 = qb * BS + wave * 32;
#pragma unroll
  for (int j = 0; j < 32 * CPR / kWave; ++j) {
    const int r = j * (kWave / CPR) + lane / CPR, c = lane % CPR;
    const u32x4_t v = *(const u32x4_t*)(ost + r * ROWB + ((c ^ (r & 15)) << 4));
    // Non-temporal: the output is not read again here, and K/V stay in L2.
    if (row0 + r < S) __builtin_nontemporal_store(v, (u32x4_t*)(obase + (int64_t)(row0 + r) * p.so[2] + c * 8));
  }
}

// Compute units of the current device (cached per device).
static int device_cus() {
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

// Resident workgroups per CU of a kernel (at least 1).
template <typename K>
static int resident_per_cu(K kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n <= 0) n = 1;
  return n;
}

template <int D, int DT>
static hipError_t launch_prefill_bs64(PrefillParams p, int* queue, hipStream_t stream) {
  const int64_t total = (int64_t)p.NB * p.B * p.Hq;
  int64_t grid = total;
  // Head dim 128 runs the two-wave kernel, one workgroup per item (measured faster than
  // the persistent ticket loop with four such workgroups per CU); head dim 64 runs the
  // four-wave one, persistent when the caller passes a workspace.
  constexpr bool two_wave = D == 128;
  constexpr int threads = two_wave ? 128 : 256;
  if constexpr (two_wave) {
    hipLaunchKernelGGL((bsfa_prefill_bs64_2w_kernel<D, DT>), dim3((unsigned)grid), dim3(threads), 0, stream, p);
  } else {
    if (queue) {
      // Every resident workgroup slot filled once, a whole number per partition.
      p.parts = (((int64_t)p.B * p.Hkv) % 8 == 0) ? 8 : 1;
      static const int per_cu = resident_per_cu(bsfa_prefill_bs64_kernel<D, DT>, threads);
      int64_t wg = std::min<int64_t>(total, (int64_t)per_cu * device_cus());
      wg = std::max<int64_t>(p.parts, wg / p.parts * p.parts);
      p.wg_per_part = (int)(wg / p.parts);
      p.queue = queue;
      grid = wg;
      hipLaunchKernelGGL(bsfa_queue_reset_kernel, dim3(1), dim3(64), 0, stream, queue);
    }
    hipLaunchKernelGGL((bsfa_prefill_bs64_kernel<D, DT>), dim3((unsigned)grid), dim3(threads), 0, stream, p);
  }
  return hipGetLastError();
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

template <int DT>
static hipError_t launch_prefill_any(const PrefillParams& p, int* queue, int64_t head_dim,
                                     int64_t block_size, hipStream_t s) {
  if (block_size == 128 && (head_dim == 128 || head_dim == 64)) {
    // A block-128 mask on the block-64 kernels: each 128-token block is its four 64-token
    // quarters, read through the mask index shift. The same tokens attend to the same
    // keys; the online softmax merely visits them in 64-key steps (2.7x faster than
    // the generic block-128 kernel at config-2 geometry).
    PrefillParams q = p;
    q.mshift = 1;
    q.NB = (p.S + 63) / 64;
    return head_dim == 128 ? launch_prefill_bs64<128, DT>(q, queue, s)
                           : launch_prefill_bs64<64, DT>(q, queue, s);
  }
  if (block_size == 64 && head_dim == 128) return launch_prefill_bs64<128, DT>(p, queue, s);
  if (block_size == 64 && head_dim == 64) return launch_prefill_bs64<64, DT>(p, queue, s);
  if (head_dim == 128) return launch_prefill<32, 128, DT>(p, s);  // block 32
  return launch_prefill<32, 64, DT>(p, s);
}

}  // namespace tasft

using namespace tasft;

static int dispatch_prefill(const PrefillParams& p, int* queue, int64_t head_dim,
                            int64_t block_size, int dtype, hipStream_t s, const char* what) {
  const hipError_t err = dtype == kF16 ? launch_prefill_any<kF16>(p, queue, head_dim, block_size, s)
                                       : launch_prefill_any<kBf16>(p, queue, head_dim, block_size, s);
  if (err != hipSuccess)
    return set_error(kErrLaunch, "%s: launch failed: %s", what, hipGetErrorString(err));
  return kOk;
}

extern "C" size_t tasft_bsfa_prefill_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                                     int64_t seq_len, int64_t block_size) {
  if (batch <= 0 || num_q_heads <= 0 || seq_len <= 0 || block_size <= 0) return 0;
  return 256;  // the persistent launch's ticket counters
}

extern "C" int tasft_bsfa_prefill_fwd(const void* q, const void* k, const void* v, void* out,
                                      const uint8_t* block_mask, void* workspace,
                                      size_t workspace_bytes, int64_t batch,
                                      int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                                      int64_t head_dim, int64_t block_size,
                                      const int64_t* q_strides, const int64_t* k_strides,
                                      const int64_t* v_strides, const int64_t* o_strides,
                                      const int64_t* mask_strides, float scale, int causal,
                                      int dtype, void* stream) {
  if (!q || !k || !v || !out || !block_mask || !q_strides || !k_strides || !v_strides ||
      !o_strides || !mask_strides)
    return set_error(kErrInvalidArgument, "prefill: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "prefill: dtype must be bf16 (0) or fp16 (1), got %d", dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0)
    return set_error(kErrInvalidArgument, "prefill: batch, heads and seq_len must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument,
                     "prefill: num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)",
                     (long long)num_q_heads, (long long)num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return set_error(kErrUnsupported, "prefill: head_dim must be 64 or 128, got %lld",
                     (long long)head_dim);
  if (block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(kErrUnsupported, "prefill: block_size must be 32, 64 or 128, got %lld",
                     (long long)block_size);
  const int64_t* st[4] = {q_strides, k_strides, v_strides, o_strides};
  if (!strides_nonneg(q_strides, 4) || !strides_nonneg(k_strides, 4) ||
      !strides_nonneg(v_strides, 4) || !strides_nonneg(o_strides, 4) ||
      !strides_nonneg(mask_strides, 4))
    return set_error(kErrInvalidArgument, "prefill: strides must be non-negative");
  for (int i = 0; i < 4; ++i) {
    if (st[i][3] != 1)
      return set_error(kErrInvalidArgument, "prefill: head_dim must be the contiguous dimension");
    for (int j = 0; j < 3; ++j)
      if (st[i][j] % 8 != 0)
        return set_error(kErrInvalidArgument,
                         "prefill: strides must be multiples of 8 elements (16-byte rows)");
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return set_error(kErrInvalidArgument, "prefill: tensors must be 16-byte aligned");
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  // Block 128 runs on the block-64 kernels (launch_prefill_any): twice the query blocks.
  if (nb * (block_size == 128 ? 2 : 1) * batch * num_q_heads > 0x7fffffffLL ||
      seq_len > 0x3fffffffLL)
    return set_error(kErrUnsupported, "prefill: problem too large for one launch");
  const size_t ws_need = tasft_bsfa_prefill_workspace_bytes(batch, num_q_heads, seq_len, block_size);
  if (workspace) {
    if (workspace_bytes < ws_need)
      return set_error(kErrWorkspace, "prefill: workspace too small: need %zu bytes, got %zu",
                       ws_need, workspace_bytes);
    if (((uintptr_t)workspace) & 15u)
      return set_error(kErrInvalidArgument, "prefill: workspace must be 16-byte aligned");
  }

  PrefillParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.o = (uint16_t*)out;
  p.mask = block_mask;
  for (int j = 0; j < 3; ++j) {
    p.sq[j] = q_strides[j];
    p.sk[j] = k_strides[j];
    p.sv[j] = v_strides[j];
    p.so[j] = o_strides[j];
  }
  for (int j = 0; j < 4; ++j) p.sm[j] = mask_strides[j];
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.S = (int)seq_len;
  p.NB = (int)nb;
  p.scale_log2 = scale * kLog2e;
  p.causal = causal ? 1 : 0;
  p.small_spans = (seq_len * k_strides[2] * 2 < 0x7fffffffLL &&
                   seq_len * v_strides[2] * 2 < 0x7fffffffLL) ? 1 : 0;
  p.queue = nullptr;
  p.parts = 1;
  p.wg_per_part = 1;
  p.cu_seqlens = nullptr;
  p.mshift = 0;
  // Ticket counters of the persistent launch (block size 64).
  return dispatch_prefill(p, (int*)workspace, head_dim, block_size, dtype, (hipStream_t)stream,
                          "prefill");
}

namespace tasft {

// Zeroes the output rows of the tokens at or after cu_seqlens[num_seqs] of a packed
// [T, H, D] batch (rows no sequence covers), reading that offset on the device: with no
// such row (the usual case) every thread makes one check and exits. Each thread writes
// 16 bytes per step; the grid strides over the tail.
__global__ void __launch_bounds__(256)
varlen_zero_tail_kernel(uint16_t* out, const int32_t* end_ptr, int64_t T, int H, int D,
                        int64_t st_t, int64_t st_h) {
  const int64_t end = *end_ptr;
  const int64_t first = end < 0 ? 0 : (end > T ? T : end);
  const int chunks = D / 8;
  const int64_t per_row = (int64_t)H * chunks;
  const int64_t n = (T - first) * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = first + i / per_row;
    const int64_t rem = i % per_row;
    const int64_t h = rem / chunks, c = rem % chunks;
    *(u32x4_t*)(out + row * st_t + h * st_h + c * 8) = (u32x4_t){0u, 0u, 0u, 0u};
  }
}

}  // namespace tasft

extern "C" int tasft_bsfa_varlen_zero_tail(void* out, const int32_t* cu_seqlens, int64_t num_seqs,
                                           int64_t tokens, int64_t num_heads, int64_t head_dim,
                                           const int64_t* o_strides, void* stream) {
  if (!out || !cu_seqlens || !o_strides)
    return set_error(kErrInvalidArgument, "varlen_zero_tail: null pointer argument");
  if (num_seqs <= 0 || tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0)
    return set_error(kErrInvalidArgument,
                     "varlen_zero_tail: num_seqs, num_heads positive, tokens >= 0, head_dim a positive multiple of 8");
  if (!strides_nonneg(o_strides, 3) || o_strides[2] != 1 || o_strides[0] % 8 != 0 ||
      o_strides[1] % 8 != 0 || !aligned16(out))
    return set_error(kErrInvalidArgument,
                     "varlen_zero_tail: out must be 16-byte aligned with a contiguous head_dim and "
                     "token and head strides multiples of 8 elements");
  if (tokens == 0) return kOk;
  hipLaunchKernelGGL(varlen_zero_tail_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream,
                     (uint16_t*)out, cu_seqlens + num_seqs, tokens, (int)num_heads, (int)head_dim,
                     o_strides[0], o_strides[1]);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "varlen_zero_tail: launch failed: %s", hipGetErrorString(err));
  return kOk;
}

extern "C" int tasft_bsfa_prefill_varlen_fwd(const void* q, const void* k, const void* v,
                                             void* out, const uint8_t* block_mask,
                                             const int32_t* cu_seqlens, int64_t num_seqs,
                                             int64_t num_q_heads, int64_t num_kv_heads,
                                             int64_t max_seqlen, int64_t head_dim,
                                             int64_t block_size, const int64_t* q_strides,
                                             const int64_t* k_strides, const int64_t* v_strides,
                                             const int64_t* o_strides,
                                             const int64_t* mask_strides, float scale, int causal,
                                             int dtype, void* stream) {
  if (!q || !k || !v || !out || !block_mask || !cu_seqlens || !q_strides || !k_strides ||
      !v_strides || !o_strides || !mask_strides)
    return set_error(kErrInvalidArgument, "prefill_varlen: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "prefill_varlen: dtype must be bf16 (0) or fp16 (1), got %d",
                     dtype);
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_seqlen <= 0)
    return set_error(kErrInvalidArgument,
                     "prefill_varlen: num_seqs, heads and max_seqlen must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument,
                     "prefill_varlen: num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)",
                     (long long)num_q_heads, (long long)num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return set_error(kErrUnsupported, "prefill_varlen: head_dim must be 64 or 128, got %lld",
                     (long long)head_dim);
  if (block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(kErrUnsupported, "prefill_varlen: block_size must be 32, 64 or 128, got %lld",
                     (long long)block_size);
  const int64_t* st[4] = {q_strides, k_strides, v_strides, o_strides};
  if (!strides_nonneg(q_strides, 3) || !strides_nonneg(k_strides, 3) ||
      !strides_nonneg(v_strides, 3) || !strides_nonneg(o_strides, 3) ||
      !strides_nonneg(mask_strides, 4))
    return set_error(kErrInvalidArgument, "prefill_varlen: strides must be non-negative");
  for (int i = 0; i < 4; ++i) {
    if (st[i][2] != 1)
      return set_error(kErrInvalidArgument,
                       "prefill_varlen: head_dim must be the contiguous dimension");
    for (int j = 0; j < 2; ++j)
      if (st[i][j] % 8 != 0)
        return set_error(kErrInvalidArgument,
                         "prefill_varlen: strides must be multiples of 8 elements (16-byte rows)");
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return set_error(kErrInvalidArgument, "prefill_varlen: tensors must be 16-byte aligned");
  const int64_t nb = (max_seqlen + block_size - 1) / block_size;
  if (nb * (block_size == 128 ? 2 : 1) * num_seqs * num_q_heads > 0x7fffffffLL ||
      max_seqlen > 0x3fffffffLL)
    return set_error(kErrUnsupported, "prefill_varlen: problem too large for one launch");

  PrefillParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.o = (uint16_t*)out;
  p.mask = block_mask;
  // Packed [tokens, heads, D]: no batch stride; the kernels add cu_seqlens[b] tokens.
  const int64_t* src[4] = {q_strides, k_strides, v_strides, o_strides};
  int64_t* dst[4] = {p.sq, p.sk, p.sv, p.so};
  for (int i = 0; i < 4; ++i) {
    dst[i][0] = 0;
    dst[i][1] = src[i][1];
    dst[i][2] = src[i][0];
  }
  for (int j = 0; j < 4; ++j) p.sm[j] = mask_strides[j];
  p.B = (int)num_seqs;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.S = (int)max_seqlen;
  p.NB = (int)nb;
  p.scale_log2 = scale * kLog2e;
  p.causal = causal ? 1 : 0;
  p.small_spans = (max_seqlen * k_strides[0] * 2 < 0x7fffffffLL &&
                   max_seqlen * v_strides[0] * 2 < 0x7fffffffLL) ? 1 : 0;
  p.queue = nullptr;
  p.parts = 1;
  p.wg_per_part = 1;
  p.cu_seqlens = cu_seqlens;
  p.mshift = 0;
  // One workgroup per (sequence, head, query block); never the persistent loop.
  return dispatch_prefill(p, nullptr, head_dim, block_size, dtype, (hipStream_t)stream,
                          "prefill_varlen");
}
