// Lightning-indexer score kernel for gfx950.
//
// Computes, per packed query row r (batch b, position s1) and key head n2,
//   score[s2] = sum_{g<G} relu(q[r, n2*G+g, :] . k[b, s2, n2, :]) * w[r, n2*G+g]
// for the visible key prefix s2 < L(s1) and writes it quantised (bf16 RNE or
// fp16) -- the arithmetic of _lightning_indexer_score_kernel
// (lightning_indexer_triton.py:180-284) and of the golden
// (lightning_indexer_numpy.py:75-92), whose quantisation happens before top-k.
//
// Mapping onto CDNA4:
//  * one wave owns one query row; the row's G heads are the MFMA M dimension
//    (MT tiles of 32 heads), keys are N (32 per MFMA), D is the contraction:
//    v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulation;
//  * the row's Q fragments stay in VGPRs for the whole key sweep (MT <= 2, MT*D <= 512),
//    otherwise they are re-read from L2 per key tile;
//  * a work-group = NW waves = NW consecutive query rows of one (batch, n2);
//    they share each K tile (64 keys for D <= 128), which is copied global ->
//    LDS by direct-to-LDS loads (no VGPR round trip) two tiles ahead into a
//    ring of three LDS buffers; one LDS-only barrier per tile, so the loads in
//    flight are never drained by it;
//  * K rows are stored unpadded with their 16-byte chunks permuted (chunk c of
//    key row k sits at c ^ (k & 15) for D >= 128), which keeps the 16-byte
//    B-fragment reads of 16 consecutive keys on distinct LDS banks;
//  * per tile a wave issues its B-fragment reads ahead of the MFMAs and keeps
//    one accumulator set per 32-key subtile, so the epilogue of one subtile can
//    overlap the MFMAs of the next;
//  * the epilogue is fused: relu(acc) * w[head] summed over the 16 heads a lane
//    holds and the MT tiles (four independent partial sums), then one
//    cross-lane add (lanes l and l^32, v_permlane32_swap) gives the per-key
//    score; the scores of a tile are written by one store at the start of the
//    next tile; fully causal-masked tiles are never loaded or computed;
//  * row blocks are issued heaviest-first (largest s1 first) to flatten the
//    causal triangle's tail.
#include <type_traits>

#include "dsa_common.hpp"

namespace dsa {

namespace {

// Tile shape (swept on the MI355X over 4 / 8 waves, 64 / 128 keys, 3 / 4 buffers: this
// setting was the fastest at C2)
constexpr int NW = 8;          // waves (= query rows) per work-group
constexpr int KEYS_PER_TILE = 64;
constexpr int RING = 3;

template <int D> struct LiTile {
  static constexpr int BN = D == 96 ? 128 : (D <= 128 ? KEYS_PER_TILE : 32);  // keys per LDS tile
  static constexpr int CPR = D / 8;                  // 16-byte chunks per key row
  // chunk permutation mask (c ^ (k & SWZ), stays in the row): 16 consecutive key rows
  // then cover 16 distinct 16-byte bank groups, conflict-free for 16-lane LDS reads
  static constexpr int SWZ = CPR % 16 == 0 ? 15 : (CPR % 8 == 0 ? 7 : 3);
  static constexpr int SLOTS = BN * CPR;             // 16-byte slots per tile
  static constexpr int IPW = SLOTS / (NW * 64);      // direct-to-LDS loads per wave per tile
  static_assert(IPW >= 1 && IPW * NW * 64 == SLOTS, "tile must split evenly over the waves");
  static constexpr int NBUF = RING;                  // LDS ring: tile t being read, the rest in flight
};

__device__ __forceinline__ float load_w(const void* w, int wdt, int64_t i) {
  if (wdt == DSA_DTYPE_F32) return reinterpret_cast<const float*>(w)[i];
  uint16_t h = reinterpret_cast<const uint16_t*>(w)[i];
  return wdt == DSA_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ int visible_len(int s1, int aq, int ak, int S2, int mode) {
  int L;
  if (mode == 3) {
    L = ak - aq + s1 + 1;
    L = L < 0 ? 0 : L;
    L = L < S2 ? L : S2;
    L = L < ak ? L : ak;
  } else {
    L = ak < S2 ? ak : S2;
  }
  return L < 0 ? 0 : L;
}

template <int IO, int D, int MT, bool PAGED>
__global__ __launch_bounds__(NW * 64) void li_score_kernel(LiScoreArgs a) {
  using T = LiTile<D>;
  constexpr int KK = D / 16;                 // MFMA k-steps
  constexpr int NSUB = T::BN / 32;           // 32-key subtiles per tile
  constexpr bool QREG = MT <= 2 && MT * D <= 512;   // Q fragments resident in VGPRs
  __shared__ __attribute__((aligned(16))) uint16_t kt[T::NBUF][T::BN * D];
  __shared__ int bt_s[PAGED ? LI_MAX_BLOCKS : 1];   // PA_BSND: the batch's block-table row

  const int lane = threadIdx.x & 63;
  // wave index in an SGPR: every per-row bound below is then wave-uniform and
  // the row/tile conditions compile to scalar branches instead of exec masks
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.z;
  const int n2 = blockIdx.y;
  // blockIdx.x = (row block, key chunk): with few row blocks (short query batches) the
  // visible keys of a row block are split over `ksplit` work-groups, each writing the
  // scores of its own tiles (no reduction: every key's score is independent)
  const int ksplit = a.key_split > 1 ? a.key_split : 1;
  const int kc = (int)blockIdx.x % ksplit;
  const int rb = (int)(gridDim.x / ksplit) - 1 - (int)blockIdx.x / ksplit;  // heaviest row block first
  const int G = a.n1 / a.n2;

  const int rows_b = a.row_start[b + 1] - a.row_start[b];
  const int aq = a.act_q[b], ak = a.act_k[b];
  const int nrows = rows_b < aq ? rows_b : aq;     // rows that produce scores
  const int s1_0 = rb * NW;
  if (s1_0 >= nrows) return;
  const int s1_last = (s1_0 + NW - 1 < nrows ? s1_0 + NW - 1 : nrows - 1);
  const int L_blk = visible_len(s1_last, aq, ak, a.s2, a.sparse_mode);  // monotone in s1
  if (L_blk <= 0) return;

  const int s1 = s1_0 + wave;
  const bool row_ok = s1 < nrows;
  const int L_row = row_ok ? visible_len(s1, aq, ak, a.s2, a.sparse_mode) : 0;
  const int64_t r = (int64_t)a.row_start[b] + (row_ok ? s1 : s1_0);

  const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (r * a.n1 + (int64_t)n2 * G) * D;
  const uint16_t* kbase = reinterpret_cast<const uint16_t*>(a.k) +
                          ((PAGED ? 0 : (int64_t)a.key_start[b]) * a.n2 + n2) * D;
  const int64_t kstride = (int64_t)a.n2 * D;
  // PA_BSND: the block-table entries of the visible keys go to LDS first (one
  // round trip before the first K loads); key t then reads physical row
  // bt[t / page] * page + t % page, and a -1 block (or one past the cache) reads
  // row 0 and its score is written as 0 -- a zero key row, as the reference's
  // de-paging produces (sparse_flash_attention_triton.py:1012-1033)
  const int page = PAGED ? a.page_bs : 1;
  const int pshift = PAGED && (page & (page - 1)) == 0 ? __builtin_ctz((unsigned)page) : -1;
  auto block_of = [&](int t) { return pshift >= 0 ? t >> pshift : t / page; };
  auto phys_row = [&](int t, bool& ok) -> int64_t {
    const int bi = block_of(t);
    const int blk = bt_s[bi];
    const int64_t p = (int64_t)blk * page + (t - bi * page);
    ok = blk >= 0 && p < a.key_rows;
    return ok ? p : 0;
  };
  if constexpr (PAGED) {
    const int nb = block_of(L_blk - 1) + 1;
    for (int i = threadIdx.x; i < nb; i += NW * 64)
      bt_s[i] = i < a.max_blocks ? a.block_table[(int64_t)b * a.max_blocks + i] : -1;
    __syncthreads();
  }

  // ---- K tile staging (started first so its latency overlaps the Q / w loads).
  // Direct-to-LDS load j of wave w fills the 64 slots [64 i, 64 i + 64) of a
  // tile, i = w * IPW + j; slot s holds chunk (s % CPR) ^ (k & SWZ) of key row
  // k = s / CPR. Every lane always issues its loads (keys past L_blk re-read the
  // last visible key, whose columns are never stored), so each wave has exactly
  // IPW loads per tile in flight and one partial vmcnt wait retires a tile.
  // When the batch's key rows span less than 4 GiB from kbase (S2 * N2 * D < 2^31)
  // the byte offset of a load is a per-lane constant plus one scalar tile offset,
  // and a full tile's loads take the SGPR-base form: one VALU add per load.
  const int ntiles_all = (L_blk + T::BN - 1) / T::BN;
  const int tiles_per = (ntiles_all + ksplit - 1) / ksplit;
  const int t0 = kc * tiles_per;                  // this work-group's tiles [t0, ntiles)
  const int ntiles = t0 + tiles_per < ntiles_all ? t0 + tiles_per : ntiles_all;
  if (t0 >= ntiles) return;
  const uint32_t ksb = (uint32_t)(a.n2 * D * 2);   // key row stride in bytes
  const bool off32 = !PAGED && (uint64_t)(uint32_t)a.s2 * ksb <= 0xFFFFFFFFull;
  int dk[T::IPW];          // key row of load j within the tile
  uint32_t dcb[T::IPW];    // byte offset of its 16-byte chunk within the row
  uint32_t doff[T::IPW];   // dk * ksb + dcb
#pragma unroll
  for (int j = 0; j < T::IPW; ++j) {
    const int slot = (wave * T::IPW + j) * 64 + lane;
    dk[j] = slot / T::CPR;
    dcb[j] = 16u * (uint32_t)((slot % T::CPR) ^ (dk[j] & T::SWZ));
    doff[j] = (uint32_t)dk[j] * ksb + dcb[j];
  }
  auto dma_part = [&](int tile, uint16_t* buf, int j) {   // load j of this wave for a tile
    if (off32 && (tile + 1) * T::BN <= L_blk) {
      lds_dma16_sbase_untracked(kbase, (uint32_t)(tile * T::BN) * ksb + doff[j], buf + (wave * T::IPW + j) * 512);
    } else {
      int s2 = tile * T::BN + dk[j];
      s2 = s2 < L_blk ? s2 : L_blk - 1;
      int64_t row = s2;
      if constexpr (PAGED) {
        bool ok;
        row = phys_row(s2, ok);
      }
      lds_dma16_untracked(reinterpret_cast<const char*>(kbase) + row * (int64_t)ksb + dcb[j],
                          buf + (wave * T::IPW + j) * 512);
    }
  };
  auto dma = [&](int tile, uint16_t* buf) {
#pragma unroll
    for (int j = 0; j < T::IPW; ++j) dma_part(tile, buf, j);
  };
#pragma unroll
  for (int j = 0; j < T::NBUF - 1; ++j) dma(t0 + j, kt[j]);

  // ---- per-row operands: Q fragments (A) and head weights
  uint4 qf[QREG ? MT : 1][QREG ? KK : 1];
  if constexpr (QREG) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 32 + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        qf[mt][kk] = (row_ok && m < G) ? ldg16(qrow + (int64_t)m * D + kk * 16 + (lane >> 5) * 8)
                                       : make_uint4(0, 0, 0, 0);
    }
  }
  // weights: one coalesced load per lane (head = lane + 64 j), then each lane
  // gathers the 16 heads it holds in the MFMA output layout with lane shuffles
  float wv[MT][16];
  {
    constexpr int WJ = (MT * 32 + 63) / 64;
    float wl[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
      const int h = lane + 64 * j;
      wl[j] = (row_ok && h < G) ? load_w(a.w, a.wdt, r * a.n1 + (int64_t)n2 * G + h) : 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int h = mt * 32 + m32_row(i, lane);
        const float v = __shfl(wl[(mt * 32) / 64], h & 63);
        wv[mt][i] = v;
      }
  }

  // Scores go out through a buffer store whose range is the row's visible keys:
  // the hardware drops every lane past L_row, and lanes of an empty slot are
  // given an offset past it, so no lane needs a compare or an exec mask.
  uint16_t* srow = a.scores + (r * a.n2 + n2) * a.ld;
  const __amdgpu_buffer_rsrc_t srd =
      __builtin_amdgcn_make_buffer_rsrc(srow, (short)0, L_row * 2, 0x00020000);
  constexpr int OOB = 1 << 30;

  // ---- main loop, software-pipelined by 32-key subtile: the MFMAs of subtile
  // j are interleaved with the relu*w epilogue of subtile j-1 (ping-pong
  // accumulators), so the wave's VALU work co-executes with its MFMAs.
  f32x16 acc[2][MT];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[u][mt][i] = 0.f;
  int pend_key0 = -1;   // first key of the subtile whose epilogue is pending (-1: none)

  // Scores of a subtile wait in a register slot and are written at the start of
  // the next tile, before its K loads are issued, so the stores never hold up
  // the partial vmcnt wait for the tile in flight. Slots pair up: lanes 0-31
  // store slot 2m, lanes 32-63 slot 2m+1 (64 consecutive keys, one store).
  constexpr int NSLOT = NSUB;
  float pv[NSLOT];
  int pk[NSLOT];
#pragma unroll
  for (int i = 0; i < NSLOT; ++i) pk[i] = -1;
  auto flush = [&]() {
#pragma unroll
    for (int m = 0; m < NSLOT; m += 2) {
      const int klo = pk[m], khi = m + 1 < NSLOT ? pk[m + 1] : -1;   // wave-uniform
      if (klo < 0 && khi < 0) continue;
      const bool hi = lane >= 32;
      float v = (hi && m + 1 < NSLOT) ? pv[m + 1] : pv[m];
      int s2;
      if (klo >= 0 && khi == klo + 32) {
        s2 = klo + lane;
      } else {
        const int kb = hi ? khi : klo;
        s2 = kb >= 0 ? kb + (lane & 31) : OOB;
      }
      if constexpr (PAGED) {
        bool ok;
        phys_row(s2 < L_row ? s2 : 0, ok);
        v = ok ? v : 0.f;
      }
      __builtin_amdgcn_raw_buffer_store_b16(from_f32<IO>(v), srd, s2 * 2, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NSLOT; ++i) pk[i] = -1;
  };
  auto finish = [&](float (&p4)[4], int key0, int slot) {
    const float p = (p4[0] + p4[1]) + (p4[2] + p4[3]);
    // lanes l and l^32 hold the two halves of the head sum of the same key
    pv[slot] = add_half_swap(p);
    pk[slot] = key0;
  };
  // Per-lane B-fragment read addresses in buffer 0, subtile 0 (rows are 8-aligned
  // per subtile, so a row's permutation key is lane & SWZ): chunk 2 kk + h sits at
  // GS * (kk / JN) + ((2 (kk % JN) + h) ^ (lane & SWZ)), h = lane >> 5. The buffer
  // and subtile offsets are compile-time in the unrolled ring below and go into the
  // reads' offset field.
  constexpr int GS = T::SWZ + 1, JN = GS / 2;
  constexpr int KC = KK < 8 ? KK : 8;              // k-steps whose fragments are read together
  const uint16_t* rp[JN];
#pragma unroll
  for (int j = 0; j < JN; ++j) rp[j] = &kt[0][(lane & 31) * D] + 8 * ((2 * j + (lane >> 5)) ^ (lane & T::SWZ));
  auto bread = [&](auto bufc, int sub, int kk) -> uint4 {
    constexpr int BUF = decltype(bufc)::value;
    return *reinterpret_cast<const uint4*>(rp[kk % JN] + BUF * T::BN * D + sub * 32 * D + 8 * GS * (kk / JN));
  };
  // MFMAs of one k-chunk into `cur` with the B fragments `bf`; the epilogue of
  // `prev` interleaved when `hp` (std::true_type / std::false_type); `hook` runs
  // after the MFMAs of the chunk's second k-step
  auto chunk = [&](auto hp, f32x16(&cur)[MT], f32x16(&prev)[MT], const uint4 (&bf)[KC], int k0, float (&p4)[4],
                   auto&& hook) {
    constexpr bool has_prev = decltype(hp)::value;
    constexpr int EPK = (MT * 16 + KK - 1) / KK;   // epilogue elements per k-step
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int kk = k0 + j;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        uint4 af;
        if constexpr (QREG) {
          af = qf[mt][kk];
        } else {
          const int m = mt * 32 + (lane & 31);
          af = (row_ok && m < G) ? ldg16(qrow + (int64_t)m * D + kk * 16 + (lane >> 5) * 8)
                                 : make_uint4(0, 0, 0, 0);
        }
        cur[mt] = Mfma<IO>::m32(af, bf[j], kk == 0 ? f32x16{} : cur[mt]);
      }
      if constexpr (has_prev) {
#pragma unroll
        for (int q = 0; q < EPK; ++q) {
          const int e = kk * EPK + q;
          if (e < MT * 16) p4[e & 3] += fmaxf(prev[e >> 4][e & 15], 0.f) * wv[e >> 4][e & 15];
        }
      }
      if (j == 1) hook();
    }
  };
  auto drain = [&](f32x16(&prev)[MT], int key0, int slot) {
    float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < MT * 16; ++e) p4[e & 3] += fmaxf(prev[e >> 4][e & 15], 0.f) * wv[e >> 4][e & 15];
    finish(p4, key0, slot);
  };

  // One tile from LDS buffer BUF = t % 3 while tile t+1 has landed (or is
  // landing) in the next buffer and tile t+2 is being loaded into the third.
  // Right after the barrier a wave first requests its first B fragments, then
  // writes the previous tile's scores (overlapping the wait for the LDS reads).
  // Its loads of tile t+2 are spread over the subtiles, load j after the second
  // k-step of subtile j % NSUB: a direct-to-LDS load holds the wave's issue for
  // tens of cycles, and issued together at the tile start they stopped both
  // waves of a SIMD at the same time (about 1% of the kernel at C2).
  auto tile_body = [&](auto bufc, int t) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr int NXT = (BUF + T::NBUF - 1) % T::NBUF;   // buffer of tile t+2: held tile t-1
    if (t * T::BN < L_row) {   // wave-uniform: this row sees part of the tile
      uint4 bf[KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) bf[j] = bread(bufc, 0, j);
      flush();            // scores of tile t-1
      if constexpr (NSUB % 2 == 0) {
#pragma unroll
        for (int sub = 0; sub < NSUB; ++sub) {
          f32x16(&cur)[MT] = acc[sub & 1];
          f32x16(&prev)[MT] = acc[(sub + 1) & 1];
          float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int k0 = 0; k0 < KK; k0 += KC) {
            if (sub > 0 || k0 > 0)
#pragma unroll
              for (int j = 0; j < KC; ++j) bf[j] = bread(bufc, sub, k0 + j);
            chunk(std::true_type{}, cur, prev, bf, k0, p4, [&]() {
              if (k0 == 0)
#pragma unroll
                for (int j = 0; j < T::IPW; ++j)
                  if (j % NSUB == sub) dma_part(t + T::NBUF - 1, kt[NXT], j);
            });
          }
          // sub 0 finishes the pending subtile of the previous tile (none at the
          // row's first tile: its zeroed accumulators give a slot that is not stored)
          finish(p4, sub == 0 ? pend_key0 : t * T::BN + (sub - 1) * 32, sub);
        }
        pend_key0 = t * T::BN + (NSUB - 1) * 32;
      } else {
        dma(t + T::NBUF - 1, kt[NXT]);
        float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < KK; k0 += KC) {
          if (k0 > 0)
#pragma unroll
            for (int j = 0; j < KC; ++j) bf[j] = bread(bufc, 0, k0 + j);
          chunk(std::false_type{}, acc[0], acc[1], bf, k0, p4, []() {});
        }
        drain(acc[0], t * T::BN, 0);
      }
    } else {
      flush();
      dma(t + T::NBUF - 1, kt[NXT]);
      if (pend_key0 >= 0) {
        drain(acc[1], pend_key0, 0);
        pend_key0 = -1;
      }
    }
    wait_vmcnt<T::IPW * (T::NBUF - 2)>();   // this wave's part of tile t+1 has landed
    lds_barrier();
  };
  static_assert(T::NBUF == 3, "the ring below is unrolled for three buffers");
  wait_vmcnt<0>();
  lds_barrier();
  for (int t = t0; t < ntiles; t += 3) {
    tile_body(std::integral_constant<int, 0>{}, t);
    if (t + 1 >= ntiles) break;
    tile_body(std::integral_constant<int, 1>{}, t + 1);
    if (t + 2 >= ntiles) break;
    tile_body(std::integral_constant<int, 2>{}, t + 2);
  }
  flush();
  if (pend_key0 >= 0) {
    drain(acc[1], pend_key0, 0);
    flush();
  }
  wait_vmcnt<0>();   // no direct-to-LDS load may outlive the work-group's LDS
}

template <int IO, int D, bool PAGED>
void launch_mt(const LiScoreArgs& a, hipStream_t s, int MT, dim3 grid, dim3 block) {
  switch (MT) {
    case 1: hipLaunchKernelGGL((li_score_kernel<IO, D, 1, PAGED>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((li_score_kernel<IO, D, 2, PAGED>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((li_score_kernel<IO, D, 4, PAGED>), grid, block, 0, s, a); break;
  }
}

template <int IO, int D>
hipError_t launch_d(const LiScoreArgs& a0, hipStream_t s, int MT) {
  LiScoreArgs a = a0;
  // Short query batches leave most CUs idle (one 8-row work-group per CU): split each row
  // block's keys over enough work-groups for ~2 per CU, keeping at least 4 tiles each.
  const int64_t blocks = (int64_t)((a.max_rows_per_batch + NW - 1) / NW) * a.n2 * a.batch;
  const int max_tiles = (a.max_kv + LiTile<D>::BN - 1) / LiTile<D>::BN;
  int ks = (int)((512 + blocks - 1) / blocks);
  ks = ks < max_tiles / 4 ? ks : max_tiles / 4;
  a.key_split = ks > 1 ? (ks < 16 ? ks : 16) : 1;
  dim3 grid((unsigned)(((a.max_rows_per_batch + NW - 1) / NW) * a.key_split), a.n2, a.batch), block(NW * 64);
  if (a.block_table)
    launch_mt<IO, D, true>(a, s, MT, grid, block);
  else
    launch_mt<IO, D, false>(a, s, MT, grid, block);
  return hipGetLastError();
}

template <int IO>
hipError_t launch_io(const LiScoreArgs& a, hipStream_t s, int MT) {
  switch (a.d) {
    case 64: return launch_d<IO, 64>(a, s, MT);
    case 96: return launch_d<IO, 96>(a, s, MT);
    case 128: return launch_d<IO, 128>(a, s, MT);
    case 256: return launch_d<IO, 256>(a, s, MT);
    case 512: return launch_d<IO, 512>(a, s, MT);
  }
  return hipErrorInvalidValue;
}

}  // namespace

}  // namespace dsa

bool li_score_supported_d(int d) { return d == 64 || d == 96 || d == 128 || d == 256 || d == 512; }

hipError_t launch_li_score(const LiScoreArgs& a, hipStream_t s) {
  const int G = a.n1 / a.n2;
  const int MT = G <= 32 ? 1 : (G <= 64 ? 2 : 4);
  if (a.max_rows_per_batch <= 0 || a.total_rows <= 0) return hipSuccess;
  return a.io == dsa::IO_BF16 ? dsa::launch_io<dsa::IO_BF16>(a, s, MT)
                              : dsa::launch_io<dsa::IO_F16>(a, s, MT);
}
