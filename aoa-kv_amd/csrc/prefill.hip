// Dense causal prefill over the paged cache, gfx950 MFMA (fp16 in, fp32 acc).
//
// Replaces BatchPrefillWithPagedKVCacheKernel (kernels/aoa_kv/kernels/include/
// prefill/prefill.cuh:688-870) for one sequence: o = softmax(q k^T / sqrt(d)) v
// with query i (position L - qo_len + i) attending keys 0 .. L - qo_len + i.
//
// Formulation: each wave owns 32 queries and computes the transposed scores
// S^T = K Q^T with v_mfma_f32_32x32x16_f16 (keys on the MFMA rows, queries on
// the columns).  In the 32x32 accumulator lane l holds column l%32, so every
// lane holds the scores of ONE query -- its own -- for 16 of the tile's 32
// keys (the other 16 sit in lane l^32).  The softmax row statistics are
// therefore per lane (plus one exchange with lane l^32), and the fp16
// probabilities already sit in the B-operand layout of O^T += V^T P^T, so P
// never goes through LDS.  Lane layouts (checked on the hardware):
//   A: lane l -> row l%32, 8 k-values;  B: lane l -> column l%32, 8 k-values,
//   A and B elements with the same (l/32, j) share a k;
//   C: register i of lane l -> row 8*(i/4) + 4*(l/32) + i%4, column l%32.
//
// Block = 4 waves = 128 queries of one head.  K and V tiles of 64 keys go
// from the paged cache straight into LDS (global_load_lds_dwordx4, no
// register staging), double-buffered so tile i+1 loads while tile i is
// computed.  Rows are 256 bytes (one key, 128 dims) with their 16-byte
// chunks permuted per row (k_swz / v_swz below), so the K reads of a wave
// and the V transpose reads hit distinct banks (no LDS bank conflicts,
// measured with SQ_LDS_BANK_CONFLICT).  Each wave
// loads 16 rows per tile: one page of 16 tokens, half a page of 32 or two
// pages of 8, so its page ids are one or two scalar loads; with pages of 1,
// 2 or 4 tokens, each lane loads the id of the page of its rows (one vector
// load per load instruction).  Either way fetched a tile ahead.  The V^T operand of O^T += V^T P^T is read from the
// row-major V tile with ds_read_b64_tr_b16: in each 16-lane group, output
// lane 4a+b receives element b of the 8-byte blocks addressed by lanes a,
// a+4, a+8, a+12 (checked on the hardware), so four lanes pointing at four
// consecutive key rows give each lane one dim of four keys.
#include "kernels.hpp"

namespace aoakv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kPfThreads = 256;
constexpr int kPfQueriesPerWave = 32;
constexpr int kPfQueriesPerBlock = 128;
constexpr int kPfTileKeys = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr uint32_t kXcds = 8;  // MI355X: 8 XCDs, workgroups dealt to them round-robin

__device__ inline floatx16 mfma32(const half8& a, const half8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// This lane's value and lane l^32's, combined: v_permlane32_swap exchanges
// the two halves of the wave in registers, where __shfl_xor would go through
// the LDS unit (ds_bpermute) and queue behind the tile reads.
__device__ inline float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// row of accumulator register i for lane group g
__device__ inline int crow(int i, int g) { return 8 * (i / 4) + 4 * g + (i % 4); }

// Chunk swizzles (16-byte chunk j of key row r sits at chunk j ^ swz(r));
// a row of D dims has CH = D / 8 chunks.  K is read as one chunk of 32
// consecutive rows per instruction: XOR with r % CH spreads them over all
// chunk positions.  V is read with the transpose read: a 16-lane group takes
// 2 adjacent chunks of 4 consecutive rows (the other group of the half-wave
// the next 2 chunks), so XOR with (CH / 4) * (r % 4) gives those chunks
// distinct positions (D = 128: 16 chunks, conflict-free as measured).
template <int CH>
__device__ inline int k_swz(int r) { return r & (CH - 1); }
template <int CH>
__device__ inline int v_swz(int r) { return (CH / 4) * (r & 3); }

// One 16-byte global -> LDS copy per lane (the lane lands at byte 16 * lane
// of `lds`).  A plain function: the builtin's operands inside the kernel
// template would be value-dependent, and the host pass then drops the
// kernel's launch stub.
__device__ inline void load_lds16(const f16* g, char* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// byte offset of 16-byte chunk j of key row r in a K tile of D-dim rows
template <int D>
__device__ inline int tile_off(int r, int j) { return r * (2 * D) + 16 * (j ^ k_swz<D / 8>(r)); }

// Tile geometry of a D-dim head (namespace-scope constants: the kernel's
// lambdas use them without capturing anything).
template <int D>
struct PfShape {
  static constexpr int kRowBytes = D * 2;                        // one key row
  static constexpr int kTileBytes = kPfTileKeys * kRowBytes;     // 16 KB at D = 128
  static constexpr int kCh = kRowBytes / 16;                     // 16-byte chunks per row
  static constexpr int kRPI = 1024 / kRowBytes;                  // rows per load instruction
  static constexpr int kKS = D / 16;                             // k-steps of the score MFMAs
  static constexpr int kDB = D / 32;                             // dim blocks of O
};

// Workgroups per CU: two at head dims 64 and 128 (64 KB of LDS and at most
// 256 registers per lane each); one at 256, whose tiles take 128 KB and whose
// O accumulators alone 128 registers (one wave per SIMD, up to 512).
template <int D>
constexpr int pf_blocks_per_cu() { return D == 256 ? 1 : 2; }

// S: tokens per page (1, 2, 4, 8, 16 or 32); D: head dim (64, 128 or 256).
template <int S, int D>
__global__ __launch_bounds__(kPfThreads, pf_blocks_per_cu<D>()) void prefill_kernel(PrefillArgs a) {
  static_assert(S == 1 || S == 2 || S == 4 || S == 8 || S == 16 || S == 32,
                "a wave's 16 rows: 16 / S pages, or half of one");
  static_assert(D == 64 || D == 128 || D == 256, "head dims of the MFMA prefill");
  using Sh = PfShape<D>;

  // two buffers of [K | V] tiles, separate objects so the compiler sees that
  // the loads into one never alias the reads of the other (no wait on them)
  __shared__ __attribute__((aligned(16))) char s_buf0[2 * Sh::kTileBytes];
  __shared__ __attribute__((aligned(16))) char s_buf1[2 * Sh::kTileBytes];
  const int tid = threadIdx.x;
  const int lane = (int)__lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane / 32;      // lane group
  const int c = lane % 32;      // query column of this lane
  const uint32_t L = a.L, Lq = a.Lq;
  const uint32_t nqt = (Lq + kPfQueriesPerBlock - 1) / kPfQueriesPerBlock;
  // XCD-aware work order.  Workgroup b runs on XCD b % 8, and each XCD has
  // its own L2, so XCD x takes the contiguous range [x * per, (x+1) * per)
  // of the head-major item list: all query tiles of a head (and of the
  // query heads that share its kv head) run on one XCD, whose L2 then holds
  // that head's K/V for all of them.  Within a head, heaviest tiles first.
  const uint32_t per = (nqt * a.Hq + kXcds - 1) / kXcds;
  const uint32_t item = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (item >= nqt * a.Hq) return;  // block-uniform: the last XCD's range is short
  const uint32_t h = item / nqt;           // query head
  const uint32_t hkv = h / (a.Hq / a.H);   // its kv head (GQA groups share K/V)
  const uint32_t qt = nqt - 1u - item % nqt;  // heaviest query tiles first
  const uint32_t off = L - Lq;                 // position of query 0
  const uint32_t npages = (L + S - 1) / S;

  const uint32_t q = qt * kPfQueriesPerBlock + wave * kPfQueriesPerWave + c;
  const bool q_live = q < Lq;
  const uint32_t qpos = q_live ? off + q : L - 1u;  // last key this query sees
  // keys this block needs: up to the last live query's position
  uint32_t qlast = qt * kPfQueriesPerBlock + kPfQueriesPerBlock - 1u;
  if (qlast >= Lq) qlast = Lq - 1u;
  const uint32_t kend = a.causal ? off + qlast + 1u : L;
  const uint32_t ntiles = (kend + kPfTileKeys - 1) / kPfTileKeys;
  // keys this wave needs (waves above the diagonal skip tiles)
  uint32_t wq_last = qt * kPfQueriesPerBlock + wave * kPfQueriesPerWave + kPfQueriesPerWave - 1u;
  if (wq_last >= Lq) wq_last = Lq - 1u;
  const uint32_t wave_kend = a.causal ? off + wq_last + 1u : L;

  // ---- this lane's query, dims 16*s + 8*g .. +8 for s < D / 16
  half8 qreg[Sh::kKS];
#pragma unroll
  for (int s = 0; s < Sh::kKS; ++s)
    qreg[s] = q_live ? *reinterpret_cast<const half8*>(a.q + ((size_t)q * a.Hq + h) * D +
                                                          16 * s + 8 * g)
                     : half8{};

  // ---- tile loader: wave w fills rows 16w .. 16w+15 of K and V (keys
  // 64 t + 16 w ..), 1 KB (Sh::kRPI rows) per instruction; lane l lands at byte
  // 16*l of its instruction's rows, i.e. row l/Sh::kCh, chunk slot l%Sh::kCh -> it
  // fetches the global chunk (l%Sh::kCh) ^ swz(row).  The page of load
  // instruction i's rows: S >= 8, id[i] (rows 0..7 of the wave one page,
  // rows 8..15 the same or, S = 8, the next); S < 8, each lane's own row's
  // page.  A page past the sequence reads the last page (its keys are
  // masked).  With S >= 8 the page table is read through the constant
  // address space: the kernel never writes it, and a scalar load keeps it
  // off the vector memory counter that the K/V tile loads are waited on with.
  constexpr int kNI = 16 / Sh::kRPI;  // load instructions per wave and tile
  struct PageIds {
    uint32_t id[kNI];
  };
  const __attribute__((address_space(4))) int32_t* kv_idx =
      (const __attribute__((address_space(4))) int32_t*)a.kv_indices;
  const int lrow = lane / Sh::kCh, lslot = lane % Sh::kCh;
  auto page_of = [&](uint32_t tile) -> PageIds {
    const uint32_t key0 = tile * kPfTileKeys + 16u * (uint32_t)wave;  // the wave's first row
    PageIds ph;
    if constexpr (S >= 8) {
      uint32_t p0 = key0 / S, p1 = (key0 + 8u) / S;
      p0 = p0 < npages ? p0 : npages - 1u;
      p1 = p1 < npages ? p1 : npages - 1u;
      const uint32_t x = (uint32_t)kv_idx[p0];
      const uint32_t y = S == 8 ? (uint32_t)kv_idx[p1] : x;
#pragma unroll
      for (int i = 0; i < kNI; ++i) ph.id[i] = Sh::kRPI * i < 8 ? x : y;
    } else {
#pragma unroll
      for (int i = 0; i < kNI; ++i) {
        uint32_t p = (key0 + (uint32_t)(Sh::kRPI * i + lrow)) / S;
        p = p < npages ? p : npages - 1u;
        ph.id[i] = (uint32_t)a.kv_indices[p];
      }
    }
    return ph;
  };
  // token slot of the wave's row 0 in its page
  const uint32_t slot0 = S == 32 ? 16u * ((uint32_t)wave % 2u) : 0u;
  auto load_tile = [&](char* buf, const PageIds& phys) {
#pragma unroll
    for (int i = 0; i < kNI; ++i) {
      const int r = 16 * wave + Sh::kRPI * i + lrow;  // row in the tile; r % 16 = Sh::kRPI i + lrow
      const uint32_t pg = phys.id[i];
      const size_t e = elem_off(a.g, pg, 0, hkv, (slot0 + (uint32_t)(r & 15)) % S);
      load_lds16(a.kv + e + 8 * (lslot ^ k_swz<Sh::kCh>(r)),
                 buf + (16 * wave + Sh::kRPI * i) * Sh::kRowBytes);
      load_lds16(a.kv + e + a.g.kv + 8 * (lslot ^ v_swz<Sh::kCh>(r)),
                 buf + Sh::kTileBytes + (16 * wave + Sh::kRPI * i) * Sh::kRowBytes);
    }
  };

  // ---- per-lane LDS offsets.  K operand (S^T = K Q^T): row ks*32 + c,
  // chunk 2s + g.  V^T operand via the transpose read: in 16-lane group G,
  // lane r = 4m + a addresses key row key0 + m, dims 32t + 16*(G%2) + 4a.
  const int vm = (lane % 16) / 4, va4 = lane % 4, vG = lane / 16;
  auto v_off = [&](int t, int key0) {
    const int row = key0 + vm;
    const int dim = 32 * t + 16 * (vG % 2) + 4 * va4;
    return row * Sh::kRowBytes + 16 * ((dim / 8) ^ v_swz<Sh::kCh>(row)) + 2 * (dim % 8);
  };

  // lane-constant byte offsets inside a tile (the loop adds the buffer base)
  int k_off[Sh::kKS], v_lo[Sh::kDB], v_hi[Sh::kDB];
#pragma unroll
  for (int s8 = 0; s8 < Sh::kKS; ++s8) k_off[s8] = tile_off<D>(c, 2 * s8 + g);  // + ks * 32 rows below
#pragma unroll
  for (int t = 0; t < Sh::kDB; ++t) {  // key0 = 4g (+ ks*32 + 16*hf below) and key0 + 8
    v_lo[t] = v_off(t, 4 * g);
    v_hi[t] = v_off(t, 4 * g + 8);
  }
  // adding whole multiples of 16 rows keeps both swizzles: offsets step by
  // 16 rows
  constexpr int kRow16 = 16 * Sh::kRowBytes;

  floatx16 acc_o[Sh::kDB];
#pragma unroll
  for (int t = 0; t < Sh::kDB; ++t) acc_o[t] = floatx16{};
  float m_run = -INFINITY, l_run = 0.f;  // running max of the unscaled scores
  const float scale = a.sm_scale * kLog2e;
  // smallest query position of this wave: tiles with every key at or below
  // it (and below L) need no mask
  const uint32_t wave_q0 = off + qt * kPfQueriesPerBlock + wave * kPfQueriesPerWave;

  // one 64-key tile from LDS buffer `tile_base`
  auto tile = [&](const lds_char* tile_base, uint32_t k0) {
    const lds_char* sK = tile_base;
    const lds_char* sV = tile_base + Sh::kTileBytes;
    // ---- S^T = K Q^T for two 32-key sub-tiles.  All K fragments of a
    // sub-tile are read before its MFMAs, and the second sub-tile's reads
    // go out before the first sub-tile's MFMAs, so no MFMA waits on a
    // just-issued LDS read.  At D = 256 (16 fragments per sub-tile) they go
    // in batches of 8, each read while the previous batch's MFMAs run, to
    // keep the registers of one wave per SIMD.
    floatx16 acc_s[2];
    if constexpr (Sh::kKS <= 8) {
      half8 kf0[Sh::kKS], kf1[Sh::kKS];
#pragma unroll
      for (int s8 = 0; s8 < Sh::kKS; ++s8)
        kf0[s8] = *reinterpret_cast<const __attribute__((address_space(3))) half8*>(sK + k_off[s8]);
#pragma unroll
      for (int s8 = 0; s8 < Sh::kKS; ++s8)
        kf1[s8] = *reinterpret_cast<const __attribute__((address_space(3))) half8*>(
            sK + k_off[s8] + 2 * kRow16);
      __builtin_amdgcn_sched_barrier(0);
      acc_s[0] = floatx16{};
#pragma unroll
      for (int s8 = 0; s8 < Sh::kKS; ++s8) acc_s[0] = mfma32(kf0[s8], qreg[s8], acc_s[0]);
      acc_s[1] = floatx16{};
#pragma unroll
      for (int s8 = 0; s8 < Sh::kKS; ++s8) acc_s[1] = mfma32(kf1[s8], qreg[s8], acc_s[1]);
    } else {
      constexpr int kB = 8;                      // fragments per batch
      constexpr int kNB = 2 * Sh::kKS / kB;      // batches per tile (both sub-tiles)
      auto kread = [&](int bt, half8 (&kf)[kB]) {  // batch bt: sub-tile bt / (kNB / 2)
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int s8 = (bt % (kNB / 2)) * kB + j;
          kf[j] = *reinterpret_cast<const __attribute__((address_space(3))) half8*>(
              sK + k_off[s8] + (bt / (kNB / 2)) * 2 * kRow16);
        }
      };
      half8 kfa[kB], kfb[kB];
      acc_s[0] = floatx16{};
      acc_s[1] = floatx16{};
      kread(0, kfa);
#pragma unroll
      for (int bt = 0; bt < kNB; bt += 2) {
        kread(bt + 1, kfb);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int s8 = (bt % (kNB / 2)) * kB + j;
          acc_s[bt / (kNB / 2)] = mfma32(kfa[j], qreg[s8], acc_s[bt / (kNB / 2)]);
        }
        if (bt + 2 < kNB) kread(bt + 2, kfa);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int s8 = ((bt + 1) % (kNB / 2)) * kB + j;
          acc_s[(bt + 1) / (kNB / 2)] = mfma32(kfb[j], qreg[s8], acc_s[(bt + 1) / (kNB / 2)]);
        }
      }
    }
    // ---- causal / length mask (only where a key can be past L or past
    // some query of the wave), running max of this query
    const bool full = k0 + kPfTileKeys <= L && (!a.causal || k0 + kPfTileKeys - 1u <= wave_q0);
    if (!full) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t key = k0 + ks * 32 + crow(i, g);
          const bool ok = key < L && (!a.causal || key <= qpos);
          acc_s[ks][i] = ok ? acc_s[ks][i] : -INFINITY;
        }
    }
    float mt = acc_s[0][0];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 16; ++i) mt = fmaxf(mt, acc_s[ks][i]);
    mt = pair_max(mt);
    // Lazy rescaling: the reference max m_run moves only when some query's
    // tile max exceeds it by more than 2^8 in probability (the first tile
    // always moves it: every query sees key 0 there).  Otherwise
    // probabilities stay <= 256, exact in fp16 relative terms, and the
    // final o = O / l divides both by the same reference.
    const bool move = __builtin_amdgcn_ballot_w64((mt - m_run) * scale > 8.f) != 0;
    const float m_new = move ? fmaxf(m_run, mt) : m_run;
    const float neg_m = -m_new * scale;
    float lt = 0.f;
    half8 pb[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // 2^((s - m) * scale); a masked score (-inf) gives 0
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(acc_s[ks][i], scale, neg_m));
        lt += p;
        pb[ks][i / 8][i % 8] = (f16)p;
      }
    }
    lt = pair_sum(lt);
    if (move) {  // the reference moved for some query: rescale
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale);  // m_run = -inf: 0
      l_run = l_run * alpha;
#pragma unroll
      for (int t = 0; t < Sh::kDB; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc_o[t][i] *= alpha;
    }
    l_run = l_run + lt;
    m_run = m_new;

    // ---- O^T += V^T P^T.  B element j of half hf of sub-tile ks is the
    // probability of key ks*32 + 16*hf + 8*(j/4) + 4*g + j%4, so the A
    // operand of lane l is dim 32t + l%32 of keys key0 .. key0+3 (j < 4)
    // and key0+8 .. key0+11 (j >= 4), key0 = ks*32 + 16*hf + 4*g.
    // the 4 fragments (8 transpose reads) of dim block t+1 are read while
    // dim block t's MFMAs run
    auto vfrags = [&](int t, half8 (&vf)[4]) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {  // kk = 2*ks + hf
        const int rows = kk * kRow16;
        const half4 lo = __builtin_bit_cast(
            half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(sV + v_lo[t] + rows)));
        const half4 hi = __builtin_bit_cast(
            half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(sV + v_hi[t] + rows)));
        vf[kk] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    half8 vfa[4], vfb[4];
    vfrags(0, vfa);
#pragma unroll
    for (int t = 0; t < Sh::kDB; t += 2) {
      vfrags(t + 1, vfb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc_o[t] = mfma32(vfa[kk], pb[kk / 2][kk % 2], acc_o[t]);
      if (t + 2 < Sh::kDB) vfrags(t + 2, vfa);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc_o[t + 1] = mfma32(vfb[kk], pb[kk / 2][kk % 2], acc_o[t + 1]);
    }
  };

  load_tile(s_buf0, page_of(0u));
  PageIds phys_next = page_of(1u);
  // two tiles per trip: even tiles in buffer 0, odd tiles in buffer 1
  for (uint32_t it = 0; it < ntiles; it += 2) {
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) {
      const uint32_t ti = it + u;
      if (ti >= ntiles) break;  // uniform
      // tile ti has landed in LDS (this wave's loads: vmcnt; the others':
      // the barrier), and every wave is done with the other buffer
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (ti + 1 < ntiles) {  // in flight during this tile's MFMAs
        load_tile(u == 0u ? s_buf1 : s_buf0, phys_next);
        phys_next = page_of(ti + 2u);
      }
      if ((ti + 1u) * kPfTileKeys > L) {  // uniform: the tile holding the sequence's end
        // rows of keys at or past L hold whatever the cache held there (the
        // last page's unwritten slots, or the last page read again): their
        // probability is exactly 0, but 0 * NaN is NaN in the MFMA, so their
        // V rows are zeroed before any wave reads them
        char* vbuf = (u == 0u ? s_buf0 : s_buf1) + Sh::kTileBytes;
        const uint32_t first_dead = L - ti * kPfTileKeys;  // < kPfTileKeys
        for (uint32_t i = first_dead * (Sh::kRowBytes / 16u) + threadIdx.x;
             i < (uint32_t)kPfTileKeys * (Sh::kRowBytes / 16u); i += kPfThreads)
          reinterpret_cast<uint4*>(vbuf)[i] = uint4{0u, 0u, 0u, 0u};
        __syncthreads();
      }
      if (ti * kPfTileKeys < wave_kend)  // wave-uniform: skip tiles above this wave's queries
        tile((const lds_char*)(u == 0u ? s_buf0 : s_buf1), ti * kPfTileKeys);
    }
  }

  // ---- o = O / l: lane holds its query's dims t*32 + crow(i, g)
  if (!q_live) return;
  const float inv_l = 1.f / l_run;
  f16* orow = a.o + ((size_t)q * a.Hq + h) * D;
#pragma unroll
  for (int t = 0; t < Sh::kDB; ++t) {
#pragma unroll
    for (int i0 = 0; i0 < 16; i0 += 4) {
      half4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (f16)(acc_o[t][i0 + r] * inv_l);
      *reinterpret_cast<half4*>(orow + t * 32 + crow(i0, g)) = v;
    }
  }
}

hipError_t launch_prefill(const PrefillArgs& a, uint32_t page_size, uint32_t head_dim,
                          hipStream_t s) {
  const uint32_t nqt = (a.Lq + kPfQueriesPerBlock - 1) / kPfQueriesPerBlock;
  const uint32_t per = (nqt * a.Hq + kXcds - 1) / kXcds;
  const dim3 grid(per * kXcds), block(kPfThreads);
#define AOAKV_PF(S_, D_)                                                     \
  if (page_size == S_ && head_dim == D_) {                                   \
    hipLaunchKernelGGL((prefill_kernel<S_, D_>), grid, block, 0, s, a);      \
    return hipGetLastError();                                                \
  }
  AOAKV_PF(1, 128)
  AOAKV_PF(2, 128)
  AOAKV_PF(4, 128)
  AOAKV_PF(8, 128)
  AOAKV_PF(16, 128)
  AOAKV_PF(32, 128)
  AOAKV_PF(1, 64)
  AOAKV_PF(2, 64)
  AOAKV_PF(4, 64)
  AOAKV_PF(8, 64)
  AOAKV_PF(16, 64)
  AOAKV_PF(32, 64)
  AOAKV_PF(1, 256)
  AOAKV_PF(2, 256)
  AOAKV_PF(4, 256)
  AOAKV_PF(8, 256)
  AOAKV_PF(16, 256)
  AOAKV_PF(32, 256)
#undef AOAKV_PF
  return hipErrorInvalidValue;
}

}  // namespace aoakv
