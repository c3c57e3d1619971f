// Fused flash attention for gfx950: O = softmax(scale * Q K^T) V per head,
// head dim 64, no causal mask, keys past T masked to -inf before the exp.
//
// Replaces the reference's attention chain RawRT.attn_chain /
// _attn_chain_dev (src/rawxrt.py:813-891: QK^T GEMM -> windowed row softmax
// -> PV GEMM through device buffers) and follows the online-softmax
// recurrence of its fused variant (kernels/attn_fused.cc:7-20,
// kernels/attn_mmul.cc:201-222): running max m, correction exp(m - m'),
// running sum l, fp32 accumulator O, one divide at the end. No score matrix
// ever reaches HBM.
//
// The reference scales q and k by hd^-1/4 each (npu_whisper_encoder.py:461);
// here the product scale^2 = 1/sqrt(hd), times log2(e), is applied once: in
// the encoder by the QKV GEMM's epilogue, to q in fp32 before its bf16
// rounding (QPRE: the kernel then reads scores in the exp2 domain straight
// from the MFMAs), and for the C ABI's raw Q to the fp32 scores. Either way
// it is the same function with one rounding less.
//
// Layout: Q, K [B*nh, Tp, 64] and Vt [B*nh, 64, Tp] bf16 (Tp = T rounded up
// to 64, pad rows/columns finite; Vt keys placed by vt_key). A workgroup owns
// 128 query rows of one head (4 waves x 32 rows) and streams 64-key K/Vt
// tiles through a 3-stage LDS ring filled by direct-to-LDS loads.
// Scores are computed transposed, S^T = K Q^T with v_mfma_f32_32x32x16_bf16,
// so a lane owns one query column and 16 keys per 32-key block: the row max
// and row sum are lane-local plus one exchange between the two lane halves,
// and the correction factor is one scalar per lane. P^T is repacked to bf16
// in registers and multiplied as O^T += V^T P^T; V^T's k-slots are read from
// LDS in exactly the key order the score fragment left in each lane.
#include <utility>

#include "common.h"
#include "kernels.h"

namespace wx {

constexpr int kQB = 128;            // query rows per workgroup (4 waves x 32)
constexpr int kKB = kAttnKeyBlock;  // keys per LDS tile
constexpr int kStages = 3;          // K/Vt tiles in flight
constexpr int kTile = kKB * 128;    // one 64 x 64 bf16 tile: 64 rows of 128 bytes

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);
}

// K tile [64 keys][64 dims] and Vt tile [64 dims][64 keys] stream through a
// kStages-deep LDS ring by buffer_load_dwordx4 ... lds (1 KB = 8 rows per
// instruction, lane l at byte 16 l). Rows are 128 bytes; 16-byte chunk c of
// row r sits in slot c ^ ((r >> 1) & 7), which makes the 16-lane groups of a
// ds_read_b128 hit 16 distinct bank units on gfx950's 64-bank LDS.
// max of a value over the lane pair (l, l ^ 32), in every lane, without
// LDS: v_permlane32_swap exchanges the upper half of one register with the
// lower half of the other, so the two results hold each lane's own value
// and its partner's.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// KSPLIT = 2 (few workgroups, e.g. batch 1): 8 waves, the k-th group of 4
// takes the k-th share of the key blocks for the same 4 x 32 queries, each
// group through its own ring; the groups' (O, max, sum) are combined
// through LDS at the end (written for any KSPLIT).
template <bool OUT_F32, int KSPLIT, bool QPRE>
__global__ __launch_bounds__(256 * KSPLIT) void attn_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ Vt, int n_head, int T, int Tp,
    float scale_log2, void* __restrict__ O, int64_t ldo) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[KSPLIT * kStages * 2 * kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  // wave index: uniform across the wave; readfirstlane makes that visible
  // to the compiler, so everything derived from it stays in SGPRs
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = w & 3, kh = w >> 2;  // query group, key part
  // the query blocks of one head run on one XCD, which then fetches that
  // head's K and Vt into its L2 once instead of once per XCD
  const int nqb = gridDim.x;
  const int pid = xcd_remap(blockIdx.x + nqb * (blockIdx.y + gridDim.y * blockIdx.z),
                            nqb * gridDim.y * gridDim.z);
  const int qb = pid % nqb;
  const int h = (pid / nqb) % n_head, b = pid / (nqb * n_head);
  const int64_t bh = (int64_t)b * n_head + h;
  const int q0 = qb * kQB + qg * 32;
  const uint16_t* Qh = Q + bh * Tp * kHeadDim;
  const uint16_t* Kh = K + bh * Tp * kHeadDim;
  const uint16_t* Vh = Vt + bh * kHeadDim * Tp;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kh, (short)0, Tp * kHeadDim * 2, 0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)Vh, (short)0, kHeadDim * Tp * 2, 0x00020000);

  // DMA: wave qg of a part moves tile rows 16 qg .. 16 qg + 15 of both tiles
  const int lrow = lane >> 3;
  uint32_t koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = (qg * 2 + j) * 8 + lrow;
    const int lchunk = (lane & 7) ^ ((row >> 1) & 7);
    koff[j] = (uint32_t)((row * kHeadDim + lchunk * 8) * 2);
    voff[j] = (uint32_t)((row * Tp + lchunk * 8) * 2);
  }
  // key blocks of this part: [kbeg, kbeg + nkb); every wave runs nb trips
  // (one barrier each), a part with fewer blocks idles through the last
  const int nkb_all = Tp / kKB;
  const int nb = (nkb_all + KSPLIT - 1) / KSPLIT;
  const int kbeg = kh * nb;
  const int nkb = max(0, min(nkb_all, kbeg + nb) - kbeg);
  uint8_t* ring = smem + kh * (kStages * 2 * kTile);
  auto issue = [&](int i) {  // the part's i-th block into slot i % kStages
    uint8_t* base = ring + (i % kStages) * 2 * kTile;
    const int kb = kbeg + i;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(base + (qg * 2 + j) * 1024), 16,
                                               koff[j], kb * kKB * kHeadDim * 2, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(base + kTile + (qg * 2 + j) * 1024),
                                               16, voff[j], kb * kKB * 2, 0, 0);
  };

  int qrow = q0 + l32;
  qrow = qrow < Tp ? qrow : Tp - 1;
  bf16x8 qf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    qf[kk] = *reinterpret_cast<const bf16x8*>(Qh + (int64_t)qrow * kHeadDim + kk * 16 + half * 8);

  f32x16 o[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  // mc: the running exp2 reference (log2 domain), set by the first block;
  // l_run: this lane's share of the row sum
  float mc = 0.f, l_run = 0.f;
  f32x16 negm, zero16;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = zero16[r] = 0.f;
  const int sw = (l32 >> 1) & 7;  // the swizzle of every row this lane reads

#pragma unroll
  for (int st = 0; st < kStages; ++st)
    if (st < nkb) issue(st);
  if (kStages - 1 < nkb)
    wait_vm<(kStages - 1) * 4>();
  else
    wait_vm<0>();
  dma_ring_barrier();

  // One 64-key block. The ring slot is a compile-time constant (the loop
  // below is unrolled by kStages), so every LDS read address is a per-lane
  // register plus an immediate offset.
  auto block = [&](int i, auto slot_c) {
    if (i >= nkb) {  // this part has run out of blocks: keep the barrier count
      wait_vm<0>();
      dma_ring_barrier();
      return;
    }
    const int kb = kbeg + i;
    constexpr int slot = decltype(slot_c)::value;
    const uint8_t* Ks = ring + slot * 2 * kTile;
    const uint8_t* Vs = Ks + kTile;
    // all 16 fragments of the tile are read up front: the K reads feed the
    // score MFMAs, the V reads land while the softmax runs
    bf16x8 ka[2][4], va[4][2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        ka[k2][kk] = *reinterpret_cast<const bf16x8*>(
            Ks + (k2 * 32 + l32) * 128 + (((kk * 2 + half) ^ sw) << 4));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < 2; ++db)
        va[ks][db] = *reinterpret_cast<const bf16x8*>(
            Vs + (db * 32 + l32) * 128 + (((ks * 2 + half) ^ sw) << 4));
    // S^T = K Q^T for two 32-key blocks. Every score leaves this section as
    // its exp2 argument a = s c - mc, with c = scale * log2(e) and mc the
    // lane's running reference (log2 domain): with a pre-scaled Q (QPRE) the
    // accumulators start from -mc (the negm block), so the MFMAs produce a
    // directly; otherwise they start from zero and one FMA per score forms it.
    f32x16 s[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      if constexpr (QPRE)
        s[k2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[k2][0], qf[0], negm, 0, 0, 0);
      else
        s[k2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[k2][0], qf[0], zero16, 0, 0, 0);
#pragma unroll
      for (int kk = 1; kk < 4; ++kk)
        s[k2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[k2][kk], qf[kk], s[k2], 0, 0, 0);
    }
    if constexpr (!QPRE) {
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[k2][r] = fmaf(s[k2][r], scale_log2, -mc);
    }
    // Keys >= T exist only in the last block: mask them there (a uniform
    // branch), nowhere else.
    if ((kb + 1) * kKB > T) {
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * kKB + k2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          if (key >= T) s[k2][r] = -INFINITY;
        }
    }
    // p = 2^(a - sub) in bf16 pairs; the block's row sum lb adds exactly
    // those bf16 values (one v_dot2_f32_bf16 per pair), the same P that
    // multiplies V
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    uint32_t pk[2][8];
    float lb;
    auto exps = [&](auto sub_c, float sub) {
      constexpr bool SUB = decltype(sub_c)::value;
      lb = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float a0 = SUB ? s[k2][2 * j] - sub : s[k2][2 * j];
          const float a1 = SUB ? s[k2][2 * j + 1] - sub : s[k2][2 * j + 1];
          pk[k2][j] = f2bf2(__builtin_amdgcn_exp2f(a0), __builtin_amdgcn_exp2f(a1));
          lb = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk[k2][j]), ones, lb,
                                               false);
        }
    };
    // No block maximum on the common path: the reference mc moves only when
    // some p of the block exceeds 2^16 (then the block's sum does, too; an
    // overflow to inf as well), which bf16 P and the fp32 sums hold without
    // loss. Then -- and on a part's first block, which sets mc from its own
    // maximum -- the block maximum is taken, mc raised by delta, O and l
    // rescaled by 2^-delta and the block's exps redone. mc is always an
    // observed maximum, so the largest score so far contributes p = 1 and l
    // never underflows. The branch is wave-uniform and after the first block
    // rarely taken.
    exps(std::false_type{}, 0.f);
    if (i == 0 || __builtin_amdgcn_ballot_w64(lb > 65536.0f) != 0) {
      float mx = -INFINITY;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[k2][r]);
      mx = max_halves(mx);
      // first block: O and l are zero, mc takes the block maximum (it may
      // fall); later: mc only rises
      const float delta = i == 0 ? mx : fmaxf(mx, 0.f);
      const float alpha = i == 0 ? 1.f : __builtin_amdgcn_exp2f(-delta);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      mc += delta;
      if constexpr (QPRE) {
#pragma unroll
        for (int r = 0; r < 16; ++r) negm[r] = -mc;
      }
      exps(std::true_type{}, delta);
    }
    l_run += lb;

    // O^T += V^T P^T, 16 keys per MFMA; Vt rows hold each lane half's 8 keys
    // contiguously (vt_key), so one 16-byte read is the whole A fragment
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int k2 = ks >> 1, sub = ks & 1;
      const u32x4 pv = {pk[k2][4 * sub + 0], pk[k2][4 * sub + 1], pk[k2][4 * sub + 2],
                        pk[k2][4 * sub + 3]};
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pv);
#pragma unroll
      for (int db = 0; db < 2; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[ks][db], pb, o[db], 0, 0, 0);
    }
    // tile kb+1 must have landed (the stages after it may still fly); every
    // wave is done with slot kb once past the barrier, which it then refills
    if (i + kStages - 1 < nkb)
      wait_vm<(kStages - 2) * 4>();
    else
      wait_vm<0>();
    dma_ring_barrier();
    if (i + kStages < nkb) issue(i + kStages);
  };
  static_assert(kStages == 3, "the unrolled loop below walks 3 slots");
  int i = 0;
  for (; i + 2 < nb; i += 3) {
    block(i, std::integral_constant<int, 0>{});
    block(i + 1, std::integral_constant<int, 1>{});
    block(i + 2, std::integral_constant<int, 2>{});
  }
  if (i < nb) block(i, std::integral_constant<int, 0>{});
  if (i + 1 < nb) block(i + 1, std::integral_constant<int, 1>{});

  {
    const auto sw2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run),
                                                      __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(sw2[0]) + __uint_as_float(sw2[1]);
  }
  if constexpr (KSPLIT > 1) {
    // Groups 1.. hand (O, max, sum) to group 0 through LDS (idle: every
    // group's last trip waited for its DMA before the last barrier):
    // O = sum_k O_k 2^(m_k - m), l likewise, m = max over the groups that
    // saw keys (a group without key blocks, T <= 64 (KSPLIT - 1), left
    // l = 0, O = 0 and is skipped).
    constexpr int kSlot = 34 * 64;  // floats per (group, query group)
    float* xs = reinterpret_cast<float*>(smem) + lane;
    if (kh > 0) {
      float* my = xs + ((kh - 1) * 4 + qg) * kSlot;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) my[(db * 16 + r) * 64] = o[db][r];
      my[32 * 64] = mc;
      my[33 * 64] = l_run;
    }
    __syncthreads();
    if (kh > 0) return;
    float mm = mc, mk[KSPLIT - 1], lk[KSPLIT - 1];
#pragma unroll
    for (int k = 0; k < KSPLIT - 1; ++k) {
      const float* src = xs + (k * 4 + qg) * kSlot;
      mk[k] = src[32 * 64];
      lk[k] = src[33 * 64];
      if (!(lk[k] == 0.f)) mm = fmaxf(mm, mk[k]);
    }
    const float a0 = __builtin_amdgcn_exp2f(mc - mm);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] *= a0;
    l_run *= a0;
#pragma unroll
    for (int k = 0; k < KSPLIT - 1; ++k) {
      const float* src = xs + (k * 4 + qg) * kSlot;
      const float ak = lk[k] == 0.f ? 0.f : __builtin_amdgcn_exp2f(mk[k] - mm);
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] += src[(db * 16 + r) * 64] * ak;
      l_run += lk[k] * ak;
    }
  }
  const float inv = 1.0f / l_run;
  const int q = q0 + l32;
  if (q >= T) return;
  const int64_t orow = ((int64_t)b * T + q) * ldo + (int64_t)h * kHeadDim;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = db * 32 + 8 * g + 4 * half;
      const float v0 = o[db][4 * g + 0] * inv, v1 = o[db][4 * g + 1] * inv;
      const float v2 = o[db][4 * g + 2] * inv, v3 = o[db][4 * g + 3] * inv;
      if (OUT_F32) {
        const f32x4 vv = {v0, v1, v2, v3};
        *reinterpret_cast<f32x4*>(static_cast<float*>(O) + orow + d0) = vv;
      } else {
        const u32x2 vv = {f2bf2(v0, v1), f2bf2(v2, v3)};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(O) + orow + d0) = vv;
      }
    }
#endif
}

hipError_t launch_attention(const uint16_t* Q, const uint16_t* K,
                            const uint16_t* Vt, int batch, int n_head, int T,
                            float scale, void* O, int o_dtype, int64_t ldo,
                            hipStream_t s, bool q_prescaled, int keysplit) {
  if (T <= 0 || batch <= 0 || n_head <= 0) return hipSuccess;
  const int Tp = attn_padded_len(T);
  dim3 grid((T + kQB - 1) / kQB, n_head, batch);
  const float scale_log2 = attn_q_scale(scale);
  // Fewer workgroups than CUs (batch 1: 20 heads x 12 query blocks): split
  // every workgroup's keys over two groups of 4 waves, halving each wave's
  // walk (-8 % at batch 1; a third group measured no faster). keysplit 1:
  // never.
  const bool few = (int64_t)grid.x * grid.y * grid.z < 256;
  const int ks = !few || keysplit == 1 ? 1 : 2;
  const bool f32 = o_dtype == DT_F32;
#define WX_ATTN(F32, KS, QP)                                                            \
  if (f32 == F32 && KS == ks && q_prescaled == QP)                                     \
    attn_kernel<F32, KS, QP><<<grid, 256 * KS, 0, s>>>(Q, K, Vt, n_head, T, Tp, scale_log2, \
                                                       O, ldo);
  WX_ATTN(true, 2, true) WX_ATTN(false, 2, true) WX_ATTN(true, 1, true) WX_ATTN(false, 1, true)
  WX_ATTN(true, 2, false) WX_ATTN(false, 2, false) WX_ATTN(true, 1, false)
  WX_ATTN(false, 1, false)
#undef WX_ATTN
  return hipGetLastError();
}

// fp32 [B*T, nh*64] q/k/v rows -> Q, K [B*nh, Tp, 64] and Vt [B*nh, 64, Tp].
__global__ __launch_bounds__(256) void pack_qkv_kernel(
    const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int64_t ld, int T, int n_head, int Tp,
    uint16_t* __restrict__ Qo, uint16_t* __restrict__ Ko,
    uint16_t* __restrict__ Vo) {
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const int d = n_head * kHeadDim;
  const int64_t src = ((int64_t)b * T + t) * ld;
  for (int n = threadIdx.x; n < d; n += 256) {
    const int h = n >> 6, dd = n & 63;
    const int64_t bh = (int64_t)b * n_head + h;
    Qo[(bh * Tp + t) * kHeadDim + dd] = f2bf(q[src + n]);
    Ko[(bh * Tp + t) * kHeadDim + dd] = f2bf(k[src + n]);
    Vo[(bh * kHeadDim + dd) * Tp + vt_key(t)] = f2bf(v[src + n]);
  }
}

hipError_t launch_pack_qkv(const float* q, const float* k, const float* v,
                           int64_t ld, int batch, int T, int n_head,
                           uint16_t* Q, uint16_t* K, uint16_t* Vt,
                           hipStream_t s) {
  if (T <= 0 || batch <= 0) return hipSuccess;
  dim3 grid(T, batch);
  pack_qkv_kernel<<<grid, 256, 0, s>>>(q, k, v, ld, T, n_head,
                                       attn_padded_len(T), Q, K, Vt);
  return hipGetLastError();
}

}  // namespace wx
