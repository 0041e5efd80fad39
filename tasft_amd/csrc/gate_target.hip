// Training-time gate target without the [B, H, S, S] score tensor.
//
// Reference semantics:
//   scores = Q K^T * scale + triu(-inf, 1)            (tasft/modules/tasft_attention.py:426-443)
//   pooled = max_pool2d(pad(scores, -inf), bs, bs)    (tasft/training/objectives.py:170-178)
//   target = softmax(pooled over the flat NB_q*NB_k grid)  (objectives.py:181-185)
// plus the additive attention mask of tasft_attention.py:445-449 (scores + mask before
// the max-pool; a key-padding row [B, S] broadcast as [:, None, None, :], or a full
// [B, 1|H, S, S] mask), and two options: a per-row softmax over key blocks (the "softmax
// over k-blocks" reading of the target that the benchmark configuration uses) and the
// clamp(+-50) / temperature variant of tasft/modules/tasft_attention.py:272-290.
//
// Kernel 1 computes each block maximum with the same S^T = K . Q^T MFMA tiling as the
// prefill kernel (v_mfma_f32_32x32x16_bf16, or _f16 for fp16 inputs; fp32 accumulation)
// and keeps only the maximum of every 64x64 tile, so the work is the QK^T half of a dense
// causal prefill and nothing of size S^2 touches HBM. Kernel 2 normalises in place.
#include "common.h"

#include "../../include/tasft_amd.h"

namespace tasft {

struct GateTargetParams {
  const uint16_t* q;
  const uint16_t* k;
  float* out;  // [B, Hq, NB, NB] contiguous
  // Additive fp32 mask (masked kernels only): element (b, h, query, key) at
  // amask[b * sam[0] + h * sam[1] + query * sam[2] + key], addressable for every query and
  // key below max(NB * block, 64 * ceil(S / 64)); strides are multiples of 4 and the base is
  // 16-byte aligned.
  const float* amask;
  int64_t sq[3], sk[3], sam[3];
  int B, Hq, Hkv, G, S, NB;
  float scale;
  int causal;
  // Block-64 kernel only: 1 when the output holds 128-token blocks. Each 64-block maximum
  // then goes by atomic max into entry (qb >> 1, kb >> 1) of the [NBO, NBO] grid, which
  // the host has filled with -inf; 0 for a block-64 output (NBO = NB).
  int pool;
  int NBO;
  // Block-64 kernels: 1 when the output holds 32-token blocks ([NBO, NBO], filled with -inf
  // by the host). Each 32 x 32 quarter of a 64 x 64 score tile is then a whole block,
  // written as it is computed.
  int fine;
};

// Float max into global memory by integer atomics: a value with the sign bit clear orders
// like its bits as a signed integer, one with it set in reverse like its bits unsigned, and
// -inf (0xff800000) is the largest unsigned pattern of any non-NaN negative value.
__device__ __forceinline__ void gt_atomic_fmax(float* a, float v) {
  const int bits = __float_as_int(v);
  if (bits >= 0)
    atomicMax((int*)a, bits);
  else
    atomicMin((unsigned int*)a, (unsigned int)bits);
}

__global__ void gate_target_fill_kernel(float* out, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = v;
}


// One 16-byte-per-lane DMA (buffer_load ... lds) of 1 KB into LDS at `dst`.
__device__ __forceinline__ void gt_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (TASFT_LDS void*)dst, 16, voff, 0, 0, 0);
}


// In-place softmax over groups of `group_len` contiguous values. Finite values are
// optionally clamped to [-clamp, clamp] first, then divided by the temperature;
// -inf entries map to 0.
__global__ void __launch_bounds__(256)
gate_target_normalize_kernel(float* data, int64_t group_len, float inv_temp, float clamp) {
  __shared__ float red[256 / kWave];
  float* x = data + (int64_t)blockIdx.x * group_len;
  const int tid = threadIdx.x;
  auto xform = [&](float v) {
    if (clamp > 0.f && v > -INFINITY) v = fminf(fmaxf(v, -clamp), clamp);
    return v * inv_temp;
  };
  float mx = -INFINITY;
  for (int64_t i = tid; i < group_len; i += 256) mx = fmaxf(mx, xform(x[i]));
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int64_t i = tid; i < group_len; i += 256) sum += expf(xform(x[i]) - mx);
  sum = wave_sum(sum);
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  sum = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.f / sum;
  for (int64_t i = tid; i < group_len; i += 256) x[i] = expf(xform(x[i]) - mx) * inv;
}


// The same softmax with the group held in registers: 1024 threads, up to 16 values each
// (groups of at most 16384, e.g. the flat 128 x 128 target of one (b, head)), so each value
// is read once and written once instead of read three times.
constexpr int kNormThreads = 1024;
constexpr int kNormRegs = 16;

__global__ void __launch_bounds__(kNormThreads)
gate_target_normalize_reg_kernel(float* data, int64_t group_len, float inv_temp, float clamp) {
  __shared__ float red[kNormThreads / kWave];
  float* x = data + (int64_t)blockIdx.x * group_len;
  const int tid = threadIdx.x;
  float v[kNormRegs];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < kNormRegs; ++r) {
    const int64_t i = tid + (int64_t)r * kNormThreads;
    float t = i < group_len ? x[i] : -INFINITY;
    if (clamp > 0.f && t > -INFINITY) t = fminf(fmaxf(t, -clamp), clamp);
    v[r] = t * inv_temp;
    mx = fmaxf(mx, v[r]);
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kNormThreads / kWave; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < kNormRegs; ++r) {
    v[r] = expf(v[r] - mx);
    sum += v[r];
  }
  sum = wave_sum(sum);
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) tot += red[w];
  const float inv = 1.f / tot;
#pragma unroll
  for (int r = 0; r < kNormRegs; ++r) {
    const int64_t i = tid + (int64_t)r * kNormThreads;
    if (i < group_len) x[i] = v[r] * inv;
  }
}

// Block size 64, scores with an additive mask (unmasked scores run the one-wave-per-head
// kernel below, 7% faster at config 5). A workgroup owns one query block of HPW query heads
// of the same KV head (the target is dense, so these heads read exactly the same K blocks)
// with WPH waves per head: with WPH = 2 (the launched form) wave (hw, w) takes head hw, query rows 32*w..+31
// and all 64 keys of every causal key block (16 MFMAs per block); with WPH = 4 it takes
// rows 32*(w&1).. and the key half 32*(w>>1).. (8 MFMAs, measured 9% slower at config 5).
// K tiles are copied HBM -> LDS once for all HPW heads by buffer_load_dwordx4 ... lds
// (16-byte XOR swizzle, rows past S arrive as zeros) into three stages with two blocks in
// flight (3% faster than two stages at config 5), one fence-free barrier per block. Each wave reduces its sub-tile to one maximum with DPP / permlane swaps (no LDS
// round trips); the WPH partial maxima of a head's block are combined one block later
// from a double-buffered LDS slot.
template <int D>
__device__ __forceinline__ int gt_swz(int r, int cc) {
  return cc ^ (D == 128 ? (r & 15) : ((r >> 1) & 7));
}

//
// MASKED adds the caller's additive mask: each wave loads the mask values of its 32 x 64
// sub-tile (float4 per lane and 4-key group) before it issues the next block's DMA, so the
// fixed DMA wait also covers them, and adds them to the scaled scores before the max.
template <int D, int HPW, bool MASKED, int DT, int WPH = 2>
__global__ void __launch_bounds__(HPW * WPH * 64)
gate_target_bs64_kernel(const GateTargetParams p) {
  constexpr int BS = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int ROWB = D * 2;
  constexpr int TILE = BS * ROWB;
  constexpr int UNITS = TILE / 1024;  // 1 KB DMA units per tile
  constexpr int NWAVES = WPH * HPW;
  constexpr int HT = WPH * kWave;  // threads per head
  // Three K stages as separate LDS variables: the compiler tells them apart, so reads of
  // one stage do not wait for the DMA into another.
  __shared__ __attribute__((aligned(1024))) uint8_t k0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t k1[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t k2[TILE];
  __shared__ float red[2][HPW][WPH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hw = wave / WPH;  // head within the workgroup
  const int w4 = wave % WPH;
  const int rh = w4 & 1, kh = WPH == 4 ? (w4 >> 1) : 0;
  const int col = lane & 31;
  const int half = lane >> 5;

  // Item order: each XCD walks one KV group at a time, longest causal rows first.
  const int chunks = p.G / HPW;
  const int64_t idx = blockIdx.x;
  const int64_t groups = (int64_t)p.B * p.Hkv;
  const int64_t per_group = (int64_t)chunks * p.NB;
  int64_t grp, r;
  if ((groups & 7) == 0) {
    const int64_t j = idx >> 3;
    grp = (idx & 7) + 8 * (j / per_group);
    r = j % per_group;
  } else {
    grp = idx / per_group;
    r = idx % per_group;
  }
  const int qslot = (int)(r / chunks);
  const int qb = p.causal ? (p.NB - 1 - qslot) : qslot;
  const int b = (int)(grp / p.Hkv);
  const int kvh = (int)(grp % p.Hkv);
  const int h = kvh * p.G + (int)(r % chunks) * HPW + hw;

  const uint16_t* qbase = p.q + b * p.sq[0] + h * p.sq[1];
  const uint16_t* kbase = p.k + b * p.sk[0] + kvh * p.sk[1];
  float* orow = p.out + (((int64_t)b * p.Hq + h) * p.NBO + (qb >> p.pool)) * p.NBO;

  const int qrow = qb * BS + rh * 32 + col;
  const bool qvalid = qrow < p.S;
  const float* mrow = MASKED ? p.amask + b * p.sam[0] + h * p.sam[1] + (int64_t)qrow * p.sam[2]
                             : nullptr;
  const float post_scale = MASKED ? 1.f : p.scale;
  u32x4_t qf[KSTEPS];
  auto load_q = [&]() {
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4_t val = {0u, 0u, 0u, 0u};
      if (qvalid) val = *(const u32x4_t*)(qbase + (int64_t)qrow * p.sq[2] + ks * 16 + half * 8);
      qf[ks] = val;
    }
  };
  // DMA units of this wave: u = wave, wave + NWAVES, ...
  constexpr int UPW = (UNITS + NWAVES - 1) / NWAVES;
  int koff[UPW];
#pragma unroll
  for (int i = 0; i < UPW; ++i) {
    const int u = wave + i * NWAVES;
    const int byte = u * 1024 + lane * 16;
    const int row = byte / ROWB, pos = (byte % ROWB) / 16;
    koff[i] = u < UNITS ? (row * (int)p.sk[2] + gt_swz<D>(row, pos) * 8) * 2 : 0;
  }
  auto issue = [&](uint8_t* kt, int kb) {
    const int key0 = kb * BS;
    const int64_t rows_left = (int64_t)(p.S - key0);
    const int64_t bytes = rows_left * p.sk[2] * 2;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kbase + (int64_t)key0 * p.sk[2]), (short)0,
        bytes > 0x7fffffff ? 0x7fffffff : (int)bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int u = wave + i * NWAVES;
      if (UNITS % NWAVES == 0 || u < UNITS) gt_dma16(rs, kt + u * 1024, koff[i]);
    }
  };
  const int krow_l = kh * 32 + col;
  // One block from stage kt: this wave's 32 x 32 (or 32 x 64) sub-tile maximum.
  constexpr int NKT = WPH == 4 ? 1 : 2;  // 32-key tiles per wave
  using f32x4_t = float __attribute__((ext_vector_type(4)));
  f32x4_t mv[NKT][4];  // mask values of this lane's keys (MASKED)
  auto load_mask = [&](int kb) {
    if constexpr (MASKED) {
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          mv[t][g4] = *(const f32x4_t*)(mrow + kb * BS + kh * 32 + 32 * t + 8 * g4 + 4 * half);
    }
  };
  auto block_max = [&](const uint8_t* kt, int kb) {
    f32x16_t s[NKT];
#pragma unroll
    for (int t = 0; t < NKT; ++t) s[t] = (f32x16_t){};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cc = ks * 2 + half;
#pragma unroll
      for (int t = 0; t < NKT; ++t) {
        const int kr = krow_l + 32 * t;
        const u32x4_t a = *(const u32x4_t*)(kt + kr * ROWB + gt_swz<D>(kr, cc) * 16);
        s[t] = mfma16<DT>(a, qf[ks], s[t]);
      }
    }
    const int key0 = kb * BS;
    if constexpr (MASKED) {
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) s[t][rr] = s[t][rr] * p.scale + mv[t][rr >> 2][rr & 3];
    }
    if ((p.causal && kb == qb) || (key0 + BS > p.S) || qb * BS + BS > p.S) {
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int key = key0 + kh * 32 + 32 * t + 8 * (rr >> 2) + 4 * half + (rr & 3);
          s[t][rr] = (!qvalid || key >= p.S || (p.causal && key > qrow)) ? -INFINITY : s[t][rr];
        }
    }
    float m = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
#pragma unroll
    for (int rr = 3; rr < 15; rr += 2) m = fmaxf(fmaxf(m, s[0][rr]), s[0][rr + 1]);
    m = fmaxf(m, s[0][15]);
    if constexpr (NKT == 2) {
      float m2 = fmaxf(fmaxf(s[1][0], s[1][1]), s[1][2]);
#pragma unroll
      for (int rr = 3; rr < 15; rr += 2) m2 = fmaxf(fmaxf(m2, s[1][rr]), s[1][rr + 1]);
      m2 = fmaxf(m2, s[1][15]);
      if (p.fine) {
        // Block-32 output: this wave's rows are query block 2 qb + rh, its key tiles t = 0, 1
        // are key blocks 2 kb + t (entries past NBO belong to no block).
        m = wave_max_dpp(m);
        m2 = wave_max_dpp(m2);
        const int r = 2 * qb + rh;
        if (lane == 0 && r < p.NBO) {
          float* o = p.out + (((int64_t)b * p.Hq + h) * p.NBO + r) * p.NBO + 2 * kb;
          o[0] = m * post_scale;
          if (2 * kb + 1 < p.NBO) o[1] = m2 * post_scale;
        }
        return 0.f;
      }
      m = fmaxf(m, m2);
    }
    return wave_max_dpp(m);
  };
  // Combine the four partial maxima of this head's block kb (slot kb & 1), scaled.
  auto store = [&](int kb) {
    if ((tid % HT) == 0 && !p.fine) {
      const float* rm = red[kb & 1][hw];
      float m = rm[0];
#pragma unroll
      for (int i = 1; i < WPH; ++i) m = fmaxf(m, rm[i]);
      // Scaling by scale > 0 before the max is exact: rounding is monotonic.
      if (p.pool)
        gt_atomic_fmax(orow + (kb >> 1), m * post_scale);
      else
        orow[kb] = m * post_scale;
    }
  };

  const int kb_end = p.causal ? qb + 1 : p.NB;
  if (!p.pool && !p.fine)
    for (int kb = kb_end + (tid % HT); kb < p.NB; kb += HT) orow[kb] = -INFINITY;
  // Three stages, two blocks in flight. Past the last block the last one is loaded again,
  // so every wave always has exactly UPWX later DMA units outstanding when it waits for a
  // block, and the wait count is a constant.
  static_assert(UNITS % NWAVES == 0, "equal DMA units per wave");
  constexpr int UPWX = UNITS / NWAVES;
  constexpr int kWaitBlock = (UPWX & 15) | ((UPWX >> 4) << 14) | 0x0070;  // vmcnt(UPWX)
  auto step = [&](int kb, const uint8_t* cur, uint8_t* nxt) {
    __builtin_amdgcn_s_waitcnt(kWaitBlock);  // this wave's DMA of block kb landed
    asm volatile("s_barrier" ::: "memory");  // every wave's; stage nxt free; red slot final
    if (kb > 0) store(kb - 1);
    load_mask(kb);
    issue(nxt, min(kb + 2, kb_end - 1));
    const float m = block_max(cur, kb);
    if (lane == 0) red[kb & 1][hw][w4] = m;
  };
  // Block 0 and the query fragments land before the loop (the compiler would otherwise
  // wait for every prefetched block at the loop entry, since the loop reads qf).
  issue(k0, 0);
  load_q();
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  issue(k1, min(1, kb_end - 1));
  for (int kb = 0; kb < kb_end; kb += 3) {
    step(kb, k0, k2);
    if (kb + 1 >= kb_end) break;
    step(kb + 1, k1, k0);
    if (kb + 2 >= kb_end) break;
    step(kb + 2, k2, k1);
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA outlives the workgroup
  asm volatile("s_barrier" ::: "memory");
  store(kb_end - 1);
}

// Unmasked scores: one wave per (head, query block), its 64 query rows as two 32-row MFMA
// column tiles. Every K fragment read from LDS feeds both row tiles, halving the LDS reads
// per MFMA of the two-waves-per-head kernel above, and the block maximum is one wave's:
// no exchange between waves. HPW heads of one KV group share each K tile (three stages,
// two blocks in flight, as above).
template <int D, int HPW, int DT>
__global__ void __launch_bounds__(HPW * 64) __attribute__((amdgpu_waves_per_eu(2)))
gate_target_bs64_w1_kernel(const GateTargetParams p) {
  constexpr int BS = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int ROWB = D * 2;
  constexpr int TILE = BS * ROWB;
  constexpr int UNITS = TILE / 1024;
  static_assert(UNITS % HPW == 0, "equal DMA units per wave");
  constexpr int UPW = UNITS / HPW;
  __shared__ __attribute__((aligned(1024))) uint8_t k0[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t k1[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t k2[TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;  // head within the workgroup
  const int col = lane & 31;
  const int half = lane >> 5;

  const int chunks = p.G / HPW;
  const int64_t idx = blockIdx.x;
  const int64_t groups = (int64_t)p.B * p.Hkv;
  const int64_t per_group = (int64_t)chunks * p.NB;
  int64_t grp, r;
  if ((groups & 7) == 0) {
    const int64_t j = idx >> 3;
    grp = (idx & 7) + 8 * (j / per_group);
    r = j % per_group;
  } else {
    grp = idx / per_group;
    r = idx % per_group;
  }
  const int qslot = (int)(r / chunks);
  const int qb = p.causal ? (p.NB - 1 - qslot) : qslot;
  const int b = (int)(grp / p.Hkv);
  const int kvh = (int)(grp % p.Hkv);
  const int h = kvh * p.G + (int)(r % chunks) * HPW + wave;

  const uint16_t* qbase = p.q + b * p.sq[0] + h * p.sq[1];
  const uint16_t* kbase = p.k + b * p.sk[0] + kvh * p.sk[1];
  float* orow = p.out + (((int64_t)b * p.Hq + h) * p.NBO + (qb >> p.pool)) * p.NBO;

  int qrow[2];
  bool qvalid[2];
  u32x4_t qf[2][KSTEPS];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    qrow[rt] = qb * BS + rt * 32 + col;
    qvalid[rt] = qrow[rt] < p.S;
  }
  auto load_q = [&]() {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        u32x4_t val = {0u, 0u, 0u, 0u};
        if (qvalid[rt]) val = *(const u32x4_t*)(qbase + (int64_t)qrow[rt] * p.sq[2] + ks * 16 + half * 8);
        qf[rt][ks] = val;
      }
  };
  // DMA units of this wave: u = wave, wave + HPW, ...
  int koff[UPW];
#pragma unroll
  for (int i = 0; i < UPW; ++i) {
    const int u = wave + i * HPW;
    const int byte = u * 1024 + lane * 16;
    const int row = byte / ROWB, pos = (byte % ROWB) / 16;
    koff[i] = (row * (int)p.sk[2] + gt_swz<D>(row, pos) * 8) * 2;
  }
  auto issue = [&](uint8_t* kt, int kb) {
    const int key0 = kb * BS;
    const int64_t bytes = (int64_t)(p.S - key0) * p.sk[2] * 2;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kbase + (int64_t)key0 * p.sk[2]), (short)0,
        bytes > 0x7fffffff ? 0x7fffffff : (int)bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < UPW; ++i) gt_dma16(rs, kt + (wave + i * HPW) * 1024, koff[i]);
  };
  // Block kb from stage kt: its maximum (or, for 32-token output blocks, the maxima of its
  // four 32 x 32 quarters), written by lane 0.
  auto block_max = [&](const uint8_t* kt, int kb) {
    f32x16_t s[2][2];  // [row tile][key tile]
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t) s[rt][t] = (f32x16_t){};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cc = ks * 2 + half;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int kr = 32 * t + col;
        const u32x4_t a = *(const u32x4_t*)(kt + kr * ROWB + gt_swz<D>(kr, cc) * 16);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) s[rt][t] = mfma16<DT>(a, qf[rt][ks], s[rt][t]);
      }
    }
    const int key0 = kb * BS;
    if ((p.causal && kb == qb) || (key0 + BS > p.S) || qb * BS + BS > p.S) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int key = key0 + 32 * t + 8 * (rr >> 2) + 4 * half + (rr & 3);
            s[rt][t][rr] = (!qvalid[rt] || key >= p.S || (p.causal && key > qrow[rt])) ? -INFINITY : s[rt][t][rr];
          }
    }
    float m[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float v = fmaxf(fmaxf(s[rt][t][0], s[rt][t][1]), s[rt][t][2]);
#pragma unroll
        for (int rr = 3; rr < 15; rr += 2) v = fmaxf(fmaxf(v, s[rt][t][rr]), s[rt][t][rr + 1]);
        m[rt][t] = fmaxf(v, s[rt][t][15]);
      }
    if (p.fine) {
      // Block-32 output: quarter (rt, t) is block (2 qb + rt, 2 kb + t); entries past NBO
      // belong to no block.
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int t = 0; t < 2; ++t) m[rt][t] = wave_max_dpp(m[rt][t]);
      if (lane == 0) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int rq = 2 * qb + rt;
          if (rq >= p.NBO) continue;
          float* o = p.out + (((int64_t)b * p.Hq + h) * p.NBO + rq) * p.NBO + 2 * kb;
          o[0] = m[rt][0] * p.scale;
          if (2 * kb + 1 < p.NBO) o[1] = m[rt][1] * p.scale;
        }
      }
      return;
    }
    // Scaling by scale > 0 after the max is exact: rounding is monotonic.
    const float mx = wave_max_dpp(fmaxf(fmaxf(m[0][0], m[0][1]), fmaxf(m[1][0], m[1][1]))) * p.scale;
    if (lane == 0) {
      if (p.pool)
        gt_atomic_fmax(orow + (kb >> 1), mx);
      else
        orow[kb] = mx;
    }
  };

  const int kb_end = p.causal ? qb + 1 : p.NB;
  if (!p.pool && !p.fine)
    for (int kb = kb_end + lane; kb < p.NB; kb += kWave) orow[kb] = -INFINITY;
  // Three stages, two blocks in flight; past the last block the last one is loaded again,
  // so every wave has exactly UPW later DMA units outstanding when it waits for a block.
  constexpr int kWaitBlock = (UPW & 15) | ((UPW >> 4) << 14) | 0x0070;  // vmcnt(UPW)
  auto step = [&](int kb, const uint8_t* cur, uint8_t* nxt) {
    __builtin_amdgcn_s_waitcnt(kWaitBlock);  // this wave's DMA of block kb landed
    asm volatile("s_barrier" ::: "memory");  // every wave's; stage nxt is free
    issue(nxt, min(kb + 2, kb_end - 1));
    block_max(cur, kb);
  };
  issue(k0, 0);
  load_q();
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  issue(k1, min(1, kb_end - 1));
  for (int kb = 0; kb < kb_end; kb += 3) {
    step(kb, k0, k2);
    if (kb + 1 >= kb_end) break;
    step(kb + 1, k1, k0);
    if (kb + 2 >= kb_end) break;
    step(kb + 2, k2, k1);
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): no DMA outlives the workgroup
}

template <int D, bool MASKED, int DT>
static hipError_t launch_blockmax_bs64(const GateTargetParams& p, hipStream_t stream) {
  const int hpw = (p.G % 4 == 0) ? 4 : (p.G % 2 == 0 ? 2 : 1);
  const int64_t grid = (int64_t)p.NB * p.B * p.Hq / hpw;
  if constexpr (!MASKED) {
    if (hpw == 4)
      hipLaunchKernelGGL((gate_target_bs64_w1_kernel<D, 4, DT>), dim3((unsigned)grid), dim3(4 * 64), 0, stream, p);
    else if (hpw == 2)
      hipLaunchKernelGGL((gate_target_bs64_w1_kernel<D, 2, DT>), dim3((unsigned)grid), dim3(2 * 64), 0, stream, p);
    else
      hipLaunchKernelGGL((gate_target_bs64_w1_kernel<D, 1, DT>), dim3((unsigned)grid), dim3(64), 0, stream, p);
    return hipGetLastError();
  }
  if (hpw == 4)
    hipLaunchKernelGGL((gate_target_bs64_kernel<D, 4, MASKED, DT>), dim3((unsigned)grid), dim3(4 * 128), 0, stream, p);
  else if (hpw == 2)
    hipLaunchKernelGGL((gate_target_bs64_kernel<D, 2, MASKED, DT>), dim3((unsigned)grid), dim3(2 * 128), 0, stream, p);
  else
    hipLaunchKernelGGL((gate_target_bs64_kernel<D, 1, MASKED, DT>), dim3((unsigned)grid), dim3(128), 0, stream, p);
  return hipGetLastError();
}

template <bool MASKED, int DT>
static hipError_t dispatch_blockmax_dt(const GateTargetParams& p, int64_t block_size,
                                       int64_t head_dim, hipStream_t s) {
  // Every block size runs the block-64 kernel: block 128 with its maxima pooled 2x2
  // (p.pool), block 32 with each wave's 32 x 32 tiles as blocks (p.fine).
  (void)block_size;
  if (head_dim == 128) return launch_blockmax_bs64<128, MASKED, DT>(p, s);
  return launch_blockmax_bs64<64, MASKED, DT>(p, s);
}

template <bool MASKED>
static hipError_t dispatch_blockmax(const GateTargetParams& p, int64_t block_size,
                                    int64_t head_dim, int dtype, hipStream_t s) {
  return dtype == kF16 ? dispatch_blockmax_dt<MASKED, kF16>(p, block_size, head_dim, s)
                       : dispatch_blockmax_dt<MASKED, kBf16>(p, block_size, head_dim, s);
}

// KL gate loss (reference TASFTObjective.compute_gate_loss, objectives.py:187-221) of one
// (batch, head) per workgroup, on its flattened NB_q * NB_k scores g and target t:
//   Z = sum_i g_i + eps,  u_i = g_i / Z + eps,
//   L = sum_i t_i (log t_i - log u_i)            (entries with t_i = 0 contribute 0),
//   dL/dg_k = (-t_k / u_k + (sum_i t_i g_i / u_i) / Z) / Z.
// loss_part[bh] receives L; grad (optional) receives inv_batch * dL/dg (the reference
// reduces with "batchmean": the sum over (b, h) divided by B).
constexpr float kKlEps = 1e-8f;

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ void __launch_bounds__(256)
gate_kl_kernel(const float* soft, const float* target, int64_t n, float inv_batch,
               float* loss_part, float* grad) {
  __shared__ float red[4];
  const int64_t bh = blockIdx.x;
  const float* g = soft + bh * n;
  const float* t = target + bh * n;
  const int tid = threadIdx.x;
  float z = 0.f;
  for (int64_t i = tid; i < n; i += 256) z += g[i];
  z = block_sum256(z, red) + kKlEps;
  const float inv_z = 1.f / z;
  float l = 0.f, s2 = 0.f;
  for (int64_t i = tid; i < n; i += 256) {
    const float ti = t[i];
    if (ti > 0.f) {
      const float gi = g[i];
      const float u = gi * inv_z + kKlEps;
      l += ti * (logf(ti) - logf(u));
      s2 += ti * gi / u;
    }
  }
  l = block_sum256(l, red);
  s2 = block_sum256(s2, red);
  if (tid == 0) loss_part[bh] = l;
  if (grad) {
    float* gr = grad + bh * n;
    const float c = s2 * inv_z;
    for (int64_t i = tid; i < n; i += 256) {
      const float ti = t[i];
      const float u = g[i] * inv_z + kKlEps;
      gr[i] = inv_batch * inv_z * (c - ti / u);
    }
  }
}


// The same loss with the (b, head)'s scores and target held in registers: 1024 threads, up
// to kKlRegs elements each (NB_q * NB_k <= 16384, i.e. 128 x 128 blocks), so each value is
// read from memory once instead of three (g) and twice (t) times.
constexpr int kKlThreads = 1024;
constexpr int kKlRegs = 16;

__device__ __forceinline__ float block_sum1024(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kKlThreads / 64; ++w) s += red[w];
  return s;
}

__global__ void __launch_bounds__(kKlThreads)
gate_kl_reg_kernel(const float* soft, const float* target, int64_t n, float inv_batch,
                   float* loss_part, float* grad) {
  __shared__ float red[kKlThreads / 64];
  const int64_t bh = blockIdx.x;
  const float* g = soft + bh * n;
  const float* t = target + bh * n;
  const int tid = threadIdx.x;
  float gv[kKlRegs], tv[kKlRegs];
  float z = 0.f;
#pragma unroll
  for (int r = 0; r < kKlRegs; ++r) {
    const int64_t i = tid + (int64_t)r * kKlThreads;
    gv[r] = i < n ? g[i] : 0.f;
    tv[r] = i < n ? t[i] : 0.f;
    z += gv[r];
  }
  z = block_sum1024(z, red) + kKlEps;
  const float inv_z = 1.f / z;
  float l = 0.f, s2 = 0.f;
#pragma unroll
  for (int r = 0; r < kKlRegs; ++r) {
    if (tv[r] > 0.f) {
      const float u = gv[r] * inv_z + kKlEps;
      l += tv[r] * (logf(tv[r]) - logf(u));
      s2 += tv[r] * gv[r] / u;
    }
  }
  l = block_sum1024(l, red);
  s2 = block_sum1024(s2, red);
  if (tid == 0) loss_part[bh] = l;
  if (grad) {
    float* gr = grad + bh * n;
    const float c = s2 * inv_z;
#pragma unroll
    for (int r = 0; r < kKlRegs; ++r) {
      const int64_t i = tid + (int64_t)r * kKlThreads;
      if (i < n) gr[i] = inv_batch * inv_z * (c - tv[r] / (gv[r] * inv_z + kKlEps));
    }
  }
}

}  // namespace tasft

using namespace tasft;

extern "C" int tasft_gate_target_fwd(const void* q, const void* k, const float* attn_mask,
                                     float* target, int64_t batch, int64_t num_q_heads,
                                     int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                                     int64_t block_size, const int64_t* q_strides,
                                     const int64_t* k_strides, const int64_t* mask_strides,
                                     float scale, int causal, int normalize, float temperature,
                                     float clamp, int dtype, void* stream) {
  if (!q || !k || !target || !q_strides || !k_strides || (attn_mask && !mask_strides))
    return set_error(kErrInvalidArgument, "gate_target: null pointer argument");
  if (dtype != kBf16 && dtype != kF16)
    return set_error(kErrUnsupported, "gate_target: dtype must be bf16 (0) or fp16 (1), got %d",
                     dtype);
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0)
    return set_error(kErrInvalidArgument, "gate_target: batch, heads and seq_len must be positive");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(kErrInvalidArgument, "gate_target: num_q_heads must be a multiple of num_kv_heads");
  if (head_dim != 64 && head_dim != 128)
    return set_error(kErrUnsupported, "gate_target: head_dim must be 64 or 128, got %lld",
                     (long long)head_dim);
  if (block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(kErrUnsupported, "gate_target: block_size must be 32, 64 or 128, got %lld",
                     (long long)block_size);
  if (normalize < 0 || normalize > 2)
    return set_error(kErrInvalidArgument, "gate_target: normalize must be 0 (flat), 1 (row) or 2 (none)");
  if (!(temperature > 0.f))
    return set_error(kErrInvalidArgument, "gate_target: temperature must be > 0");
  const int64_t* st[2] = {q_strides, k_strides};
  if (!strides_nonneg(q_strides, 4) || !strides_nonneg(k_strides, 4))
    return set_error(kErrInvalidArgument, "gate_target: strides must be non-negative");
  for (int i = 0; i < 2; ++i) {
    if (st[i][3] != 1)
      return set_error(kErrInvalidArgument, "gate_target: head_dim must be the contiguous dimension");
    for (int j = 0; j < 3; ++j)
      if (st[i][j] % 8 != 0)
        return set_error(kErrInvalidArgument, "gate_target: strides must be multiples of 8 elements");
  }
  if ((((uintptr_t)q) & 15u) || (((uintptr_t)k) & 15u))
    return set_error(kErrInvalidArgument, "gate_target: tensors must be 16-byte aligned");
  if (attn_mask) {
    if (((uintptr_t)attn_mask) & 15u)
      return set_error(kErrInvalidArgument, "gate_target: attn_mask must be 16-byte aligned");
    for (int j = 0; j < 3; ++j)
      if (mask_strides[j] < 0 || mask_strides[j] % 4 != 0)
        return set_error(kErrInvalidArgument,
                         "gate_target: attn_mask strides must be non-negative multiples of 4");
  }
  const int64_t nb = (seq_len + block_size - 1) / block_size;
  // Blocks 128 and 32 run over 64-token blocks: one workgroup per 64-block row and head
  // group (a block-32 mask is read up to a multiple of 64 rows and keys).
  const int pool = block_size == 128 ? 1 : 0;
  const int fine = block_size == 32 ? 1 : 0;
  const int64_t nb_run = pool || fine ? (seq_len + 63) / 64 : nb;
  if (nb_run * batch * num_q_heads > 0x7fffffffLL)
    return set_error(kErrUnsupported, "gate_target: problem too large for one launch");

  GateTargetParams p;
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.out = target;
  p.amask = attn_mask;
  for (int j = 0; j < 3; ++j) {
    p.sq[j] = q_strides[j];
    p.sk[j] = k_strides[j];
    p.sam[j] = attn_mask ? mask_strides[j] : 0;
  }
  p.B = (int)batch;
  p.Hq = (int)num_q_heads;
  p.Hkv = (int)num_kv_heads;
  p.G = (int)(num_q_heads / num_kv_heads);
  p.S = (int)seq_len;
  p.NB = (int)nb_run;
  p.scale = scale;
  p.causal = causal ? 1 : 0;
  p.pool = pool;
  p.NBO = (int)nb;
  p.fine = fine;

  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  if (pool || fine) {
    const int64_t n = batch * num_q_heads * nb * nb;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(gate_target_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, s, target,
                       n, -INFINITY);
    if ((err = hipGetLastError()) != hipSuccess)
      return set_error(kErrLaunch, "gate_target: fill launch failed: %s", hipGetErrorString(err));
  }
  err = attn_mask ? dispatch_blockmax<true>(p, block_size, head_dim, dtype, s)
                             : dispatch_blockmax<false>(p, block_size, head_dim, dtype, s);
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate_target: block-max launch failed: %s", hipGetErrorString(err));

  if (normalize != 2) {
    const int64_t groups = normalize == 0 ? batch * num_q_heads : batch * num_q_heads * nb;
    const int64_t len = normalize == 0 ? nb * nb : nb;
    if (len > 1024 && len <= (int64_t)kNormThreads * kNormRegs)
      hipLaunchKernelGGL(gate_target_normalize_reg_kernel, dim3((unsigned)groups), dim3(kNormThreads), 0,
                         s, target, len, 1.f / temperature, clamp);
    else
      hipLaunchKernelGGL(gate_target_normalize_kernel, dim3((unsigned)groups), dim3(256), 0, s,
                         target, len, 1.f / temperature, clamp);
    if ((err = hipGetLastError()) != hipSuccess)
      return set_error(kErrLaunch, "gate_target: normalize launch failed: %s", hipGetErrorString(err));
  }
  return kOk;
}

extern "C" int tasft_gate_kl_fwd(const float* gate_scores, const float* target, int64_t batch,
                                 int64_t num_heads, int64_t num_blocks_q, int64_t num_blocks_k,
                                 float* loss_partials, float* grad_scores, void* stream) {
  if (!gate_scores || !target || !loss_partials)
    return set_error(kErrInvalidArgument, "gate_kl: null pointer argument");
  if (batch <= 0 || num_heads <= 0 || num_blocks_q <= 0 || num_blocks_k <= 0)
    return set_error(kErrInvalidArgument, "gate_kl: sizes must be positive");
  if (batch * num_heads > 0x7fffffffLL)
    return set_error(kErrUnsupported, "gate_kl: problem too large for one launch");
  const int64_t n = num_blocks_q * num_blocks_k;
  if (n <= (int64_t)kKlThreads * kKlRegs)
    hipLaunchKernelGGL(gate_kl_reg_kernel, dim3((unsigned)(batch * num_heads)), dim3(kKlThreads), 0,
                       (hipStream_t)stream, gate_scores, target, n, 1.f / (float)batch,
                       loss_partials, grad_scores);
  else
    hipLaunchKernelGGL(gate_kl_kernel, dim3((unsigned)(batch * num_heads)), dim3(256), 0,
                       (hipStream_t)stream, gate_scores, target, n, 1.f / (float)batch,
                       loss_partials, grad_scores);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(kErrLaunch, "gate_kl: launch failed: %s", hipGetErrorString(err));
  return kOk;
}
