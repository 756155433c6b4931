// Big-tile MFMA engine: 256 x 256 x BKT block tiles computed by 4 waves of
// 128 x 128, one wave per SIMD.
//
// Why 4 waves of 128 x 128: a wave's LDS fragment reads per MFMA fall with
// the size of its output tile.  A 128 x 128 wave tile reads 4 A + 4 B
// fragments per 16 MFMAs (0.5 per MFMA); the 64 x 128 wave tiles of 8 waves
// read 2 + 4 per 8 (0.75), which with the LDS-DMA writes held the LDS port,
// not the matrix cores, as the limit (MFMA busy 63% on MI355X).  The 256
// fp32 accumulators per lane need the whole AGPR file, so each SIMD holds
// exactly one wave (512 registers: 256 VGPRs + 256 AGPRs).
//
// With one wave per SIMD nothing else covers a stall, so the main loop keeps
// the matrix core fed across K-tile boundaries:
//   * fragments are double-buffered in registers: the reads of k-step ks+1
//     are interleaved 1 : 2 with the MFMAs of k-step ks;
//   * the workgroup barrier of each K tile sits before the tile's LAST
//     k-step (whose fragments are already in registers), so the barrier, the
//     first fragment reads of the next tile and the DMA issue for the freed
//     LDS slot all overlap that k-step's MFMAs instead of draining the pipe;
//   * global -> LDS moves by LDS-DMA (buffer_load ... lds) into an NSTAGE ring
//     of K tiles, NSTAGE - 1 tiles ahead of the MFMAs.  A DMA whose tile does
//     not exist is still issued, with every offset out of range (the hardware
//     returns zeros without a fetch), so the instruction stream has no branch.
#pragma once

#include "gemm_core.h"
#include "gemm_w4_epi.h"

namespace fgemm {

constexpr int SG_VMEM_READ = 0x020;

// s_waitcnt vmcnt <= N and lgkmcnt == 0 (expcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Bare workgroup barrier (no release fence: __syncthreads() would make the
// compiler wait for every outstanding LDS-DMA, vmcnt(0)).  The empty asm
// statements keep LDS accesses from moving across it at compile time.
__device__ __forceinline__ void bare_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS-DMA loader of one 256-row K-contiguous operand tile for the 4-wave
// engine.  As DmaLoader (XOR-swizzled 16-byte chunks, OOB offsets read
// zeros), but the segment-tail mask is a per-lane select instead of a
// branch, so that the DMA issue can be interleaved with MFMAs.
template <int BKT, bool DUAL>
struct W4Loader {
  static constexpr int BROWS = 256, NT = 256;
  static constexpr int RB = BKT * 2;          // LDS bytes per row
  static constexpr int CPR = RB / 16;         // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per wave instruction
  static constexpr int IPW = BROWS / RPI / 4; // instructions per wave per tile
  static_assert(!DUAL || RPI <= 32, "dual: an instruction's rows inside one 32-row group");
  uint32_t voff[IPW];  // byte offset of this lane's chunk in the panel (OOB = zero-fill)
  const char* base[2];
  int64_t ld_bytes;
  int kch[2];          // first k of this lane's chunk, by instruction parity
  int64_t k_split;     // dual: gate rows k < k_split, up rows k >= k_split (0: none)

  // 32-row groups alternate gate / up.  A wave's rows are a whole number of
  // 64-row pairs, so the pointer an instruction reads depends on j alone:
  // a compile-time choice (computed from the wave index, the compiler kept
  // both descriptors in a scratch array and issued every DMA through a
  // waterfall loop with vmcnt(0): the dual GEMM ran 2.6x slower).
  static_assert((IPW * RPI) % 64 == 0, "wave slab = whole gate/up group pairs");
  static __device__ __forceinline__ constexpr int sel_of(int j) { return DUAL ? ((j * RPI) / 32) % 2 : 0; }

  template <class RowSrc>
  __device__ __forceinline__ void setup(const void* p0, const void* p1, int64_t ld, int64_t panel_off,
                                        RowSrc row_src, int64_t ksplit = 0) {
    ld_bytes = ld * 2;
    k_split = DUAL ? ksplit : 0;
    const int64_t pan = panel_off * ld_bytes;
    base[0] = p0 ? (const char*)p0 + pan : nullptr;
    // (up rows: k is counted from the segment start, their column is k - k_split;
    // every lane that reads them has k >= k_split, so no address before p1 is read)
    base[1] = DUAL ? (p1 ? (const char*)p1 + pan - k_split * 2 : nullptr) : base[0];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    // A lane's chunk depends on its instruction only through the parity of
    // the instruction's first row / RPI (BKT 64: swz = (row >> 1) & 7 with 8
    // rows per instruction; BKT 32: not at all), so two values cover it.
    static_assert(IPW % 2 == 0, "instruction parity = j parity");
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int q = (wave * IPW + j) * RPI + lane / CPR;   // tile row
      const int chunk = (lane % CPR) ^ swz<BKT>(q);        // source chunk of LDS slot lane % CPR
      const int sel = sel_of(j);
      const int64_t row = base[sel] ? row_src(q, sel) : -1;
      voff[j] = row < 0 ? OOB : (uint32_t)(row * ld_bytes + chunk * 16);
      if (j < 2) kch[j] = chunk * 8;
    }
  }

  // Buffer resources and tail masks of one K-tile DMA at k0 (kvalid valid
  // k; <= 0: every chunk reads zeros); load_one issues instruction j of it.
  struct Prep {
    __amdgpu_buffer_rsrc_t r0, r1;
    bool kin[2][2];  // [gate / up rows][instruction parity]
  };
  __device__ __forceinline__ Prep prep(int64_t k0, int64_t kvalid) const {
    Prep p;
    p.r0 = make_rsrc(base[0] + k0 * 2);
    p.r1 = make_rsrc(base[1] + k0 * 2);
    const int64_t ks = k_split - k0;  // the split in tile coordinates
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      p.kin[0][par] = kch[par] < kvalid && (k_split == 0 || kch[par] < ks);
      p.kin[1][par] = kch[par] < kvalid && kch[par] >= ks;
    }
    return p;
  }
  __device__ __forceinline__ void load_one(const Prep& p, int j, char* dst) const {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t off = p.kin[sel_of(j)][j % 2] ? voff[j] : OOB;
    // (the resource goes through a local: passed to the builtin as a
    // conditional of two struct members, hipcc's host pass emitted the
    // launch stub of the first instantiation of the kernel only)
    const __amdgpu_buffer_rsrc_t r = sel_of(j) ? p.r1 : p.r0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r,
                                             (__attribute__((address_space(3))) void*)(dst + (wave * IPW + j) * 1024),
                                             16, off, 0, 0, 0);
  }
};

// Ring of NHALF half-slots of 32 KB (256 rows x 64 k of one operand).  K
// tile x keeps A in half-slot (2x) % NHALF and B in (2x + 1) % NHALF.  With
// NHALF = 5 (160 KB) the barrier of iteration t frees tile t's two halves,
// which take B of tile t+2 and A of tile t+3: the copy engine always has the
// older half of the next tile in flight when new work arrives, so the L2 ->
// LDS stream never drains (with two whole-tile stages every period paid the
// copy time plus the L2 latency: 811 against ~610 us on the 8192 x 4096 x
// 14336 product, MI355X).
constexpr int W4_NHALF = 5;
constexpr int W4_HALF = 256 * 64 * 2;  // bytes per half-slot

template <int BMODE, int EPI, bool STAGED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_w4_kernel(GemmArgs args) {
  constexpr int BM = 256, BN = 256, WAVES_M = 2, WAVES_N = 2, BKT = 64;
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;  // 128 x 128 per wave
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int KS = BKT / 16;                         // k-steps per K tile
  constexpr int RB = BKT * 2;                          // LDS bytes per row
  constexpr int NH = W4_NHALF;
  static_assert(KS % 2 == 0, "an even number of k-steps per tile keeps the fragment slots static");
  constexpr int RING = NH * W4_HALF;
  static_assert(RING >= W4_STAGE_BYTES && RING >= W4_DUAL_BYTES, "the staged epilogue reuses the ring");
  constexpr int SMEM = RING;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  const int64_t M = args.M;
  constexpr int OUT_BN = (BMODE == B_DUAL) ? BN / 2 : BN;
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t tiles_n = (args.N + OUT_BN - 1) / OUT_BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, tmi, tni, args);
  const int64_t m0 = (int64_t)tmi * BM;
  const int64_t n0 = (int64_t)tni * OUT_BN;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int wm = wave % WAVES_M;
  const int wn = wave / WAVES_M;

  int seg_tiles[MAX_SEGS];
  int total_tiles = 0;
  for (int s = 0; s < args.n_segs; ++s) {
    const Seg& sg = args.segs[s];
    const bool active = sg.n_hi > n0 && sg.n_lo < n0 + OUT_BN;
    seg_tiles[s] = active ? (int)((sg.k + BKT - 1) / BKT) : 0;
    total_tiles += seg_tiles[s];
  }
  const int per = (total_tiles + args.split_k - 1) / args.split_k;
  const int t_begin = blockIdx.z * per;
  const int t_end = min(total_tiles, t_begin + per);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  using LoaderA = W4Loader<BKT, false>;
  using LoaderB = W4Loader<BKT, BMODE == B_DUAL>;
  using PrepA = typename LoaderA::Prep;
  using PrepB = typename LoaderB::Prep;
  LoaderA la;
  LoaderB lb;
  PrepA pa_cur;  // A of tile t+2 (dst half-slot ha_dst)
  PrepB pb_cur;  // B of tile t+1 (dst half-slot hb_dst)
  auto setup_a = [&](int s) {
    const Seg& sg = args.segs[s];
    la.setup(sg.a, sg.a, sg.lda, m0, [&](int q, int) -> int64_t { return m0 + q < M ? q : -1; });
  };
  auto setup_b = [&](int s) {
    const Seg& sg = args.segs[s];
    if constexpr (BMODE == B_DUAL) {
      lb.setup(sg.b, sg.b2, sg.ldb, n0, [&](int q, int) -> int64_t {
        const int t4 = (q % 128) / 32;
        const int rel = (q / 128) * 64 + (t4 / 2) * 32 + q % 32;
        return n0 + rel < args.N ? rel : -1;
      }, sg.k_split);
    } else {
      const int64_t off = n0 - sg.n_lo;
      lb.setup(sg.b, sg.b, sg.ldb, off, [&](int q, int) -> int64_t {
        const int64_t n = n0 + q;
        return (n < args.N && n >= sg.n_lo && n < sg.n_hi) ? q : -1;
      });
    }
  };
  // A and B walk the flat K-tile list [t_begin, t_end) with cursors of their
  // own: A runs one tile ahead of B in the ring's issue order.
  struct Cursor {
    int s, t, n;    // segment, tile inside it, tiles in it
    int64_t k;      // the segment's K
  };
  Cursor ca, cb;
  {
    int s = 0, t = t_begin, acc_t = 0;
    while (s < args.n_segs && t >= acc_t + seg_tiles[s]) { acc_t += seg_tiles[s]; ++s; }
    ca.s = cb.s = s;
    ca.t = cb.t = t - acc_t;
    ca.n = cb.n = 0;
    ca.k = cb.k = 0;
  }
  // first = the cursor's current tile (set up its segment); else the next one
  auto advance = [&](Cursor& c, bool first, bool is_a) {
    if (!first) {
      ++c.t;
      if (c.t < c.n) return;
      do { ++c.s; } while (seg_tiles[c.s] == 0);
      c.t = 0;
    }
    c.n = seg_tiles[c.s];
    c.k = args.segs[c.s].k;
    if (is_a) setup_a(c.s);
    else setup_b(c.s);
  };

  constexpr int IPH = LoaderA::IPW;  // DMA instructions per wave per half-tile
  static_assert(IPH == LoaderB::IPW, "equal halves");
  // DMA of one half (the cursor's K tile of A or B); valid = false issues
  // the same instructions with every chunk out of range (zeros, no fetch),
  // so the instruction stream has no branch
  auto prep_a = [&](bool valid, PrepA& out) {
    const int64_t k0 = (int64_t)ca.t * BKT;
    out = la.prep(k0, valid ? ca.k - k0 : 0);
  };
  auto prep_b = [&](bool valid, PrepB& out) {
    const int64_t k0 = (int64_t)cb.t * BKT;
    out = lb.prep(k0, valid ? cb.k - k0 : 0);
  };
  auto half_ptr = [&](int h) { return smem + h * W4_HALF; };

  // per-lane fragment offsets: row (wave tile + lane % 32), chunk 2 ks + lane / 32, swizzled
  const int g = swz<BKT>(lane % 32) ^ (lane / 32);  // chunk ^ swz = 2 ks ^ g
  const int a_row = (wm * TM + lane % 32) * RB;
  const int b_row = (wn * TN + lane % 32) * RB;
  bf16x8 af[2][FM], bfr[2][FN];
  // fragment read `idx` of k-step ks of the tile in half-slots (ha, hb) into
  // register slot sl, in the order the MFMAs consume them: A0, B0 .. B3, A1 .. A3
  auto frag_read = [&](const char* pa, const char* pb, int ks, int sl, int idx) {
    const int ko = ((2 * ks) ^ g) << 4;
    if (idx == 0) af[sl][0] = *reinterpret_cast<const bf16x8*>(pa + a_row + ko);
    else if (idx <= FN) bfr[sl][idx - 1] = *reinterpret_cast<const bf16x8*>(pb + b_row + (idx - 1) * 32 * RB + ko);
    else af[sl][idx - FN] = *reinterpret_cast<const bf16x8*>(pa + a_row + (idx - FN) * 32 * RB + ko);
  };
  // MFMAs 2p and 2p+1 of a k-step, (i, j) row-major.  The operands are
  // swapped (block (i, j) is computed as B_j A_i^T), so a lane accumulates
  // four consecutive output columns of one row (the layout gemm_w4_epi.h
  // stages with 8-byte writes).
  auto mfma_pair = [&](int sl, int p) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int m = 2 * p + u, i = m / FN, j = m % FN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[sl][j], af[sl][i], acc[i][j], 0, 0, 0);
    }
  };
  constexpr int NPAIR = FM * FN / 2;  // 8 MFMA pairs per k-step ...
  static_assert(NPAIR == FM + FN, "... and 8 fragment reads: one per pair");

  // DMA spread: every k-step issues 4 DMA instructions per wave (one after
  // every other MFMA pair), so no k-step carries a burst (16 in one k-step
  // held the in-order issue: loop time per K tile 3300 cycles against the
  // MFMAs' 2048).  Per period (barrier(t-1) .. barrier(t)): last k-step of
  // tile t-1 and k-step 0 of tile t: B of tile t+1 (its deadline is
  // barrier(t)); k-steps 1 and 2 of tile t: A of tile t+2 (deadline
  // barrier(t+1)).
  static_assert(KS == 4 && IPH == 8 && NPAIR == 8, "4 DMA instructions per k-step");
  const int n_t = t_end - t_begin;
  if (n_t > 0) {
    // prologue: A0, B0, A1 whole and the first half of B1's instructions
    // into half-slots 0 .. 3; B1's rest and A2 follow in tile 0's k-steps
    advance(ca, true, true);
    advance(cb, true, false);
    prep_a(true, pa_cur);
#pragma unroll
    for (int d = 0; d < IPH; ++d) la.load_one(pa_cur, d, half_ptr(0));
    prep_b(true, pb_cur);
#pragma unroll
    for (int d = 0; d < IPH; ++d) lb.load_one(pb_cur, d, half_ptr(1));
    if (1 < n_t) advance(ca, false, true);
    prep_a(1 < n_t, pa_cur);
#pragma unroll
    for (int d = 0; d < IPH; ++d) la.load_one(pa_cur, d, half_ptr(2));
    if (1 < n_t) advance(cb, false, false);
    prep_b(1 < n_t, pb_cur);
#pragma unroll
    for (int d = 0; d < IPH / 2; ++d) lb.load_one(pb_cur, d, half_ptr(3));
    if (2 < n_t) advance(ca, false, true);
    prep_a(2 < n_t, pa_cur);
    char* hb_dst = half_ptr(3);
    char* ha_dst = half_ptr(4);
    wait_vm_lgkm0<IPH + IPH / 2>();  // tile 0 (halves 0, 1) landed (this wave's part)
    bare_barrier();
#pragma unroll
    for (int p = 0; p < NPAIR; ++p) frag_read(half_ptr(0), half_ptr(1), 0, 0, p);
    // nothing but these reads outstanding at the loop entry, so the waits
    // inside the loop can count them precisely
    wait_vm_lgkm0<63>();
    int ha = 0;  // half-slot of tile t's A (B is the next one)
    for (int t = 0; t < n_t; ++t) {
      const int hb = ha + 1 == NH ? 0 : ha + 1;
      const char* pa_t = half_ptr(ha);
      const char* pb_t = half_ptr(hb);
      // Program order is pinned (sched_barrier): each MFMA pair is followed
      // by one fragment read of the next k-step and, after every other pair,
      // by one DMA instruction, all issued in the MFMAs' shadow.
#pragma unroll
      for (int ks = 0; ks + 1 < KS; ++ks) {
#pragma unroll
        for (int p = 0; p < NPAIR; ++p) {
          mfma_pair(ks & 1, p);
          if (p % 2) {
            const int q = p / 2;
            if (ks == 0) lb.load_one(pb_cur, IPH / 2 + q, hb_dst);
            else la.load_one(pa_cur, (ks - 1) * (IPH / 2) + q, ha_dst);
          }
          frag_read(pa_t, pb_t, ks + 1, (ks + 1) & 1, p);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // Last k-step: its fragments are in registers.  Wait until this wave's
      // reads of tile t are done and its part of tile t+1 has landed (A of
      // tile t+2 may stay in flight), then one barrier: after it tile t+1 is
      // whole in LDS and tile t's half-slots (ha, hb) are free for B of tile
      // t+2 and A of tile t+3.
      const bool b_more = t + 2 < n_t, a_more = t + 3 < n_t;
      if (b_more) advance(cb, false, false);
      if (a_more) advance(ca, false, true);
      wait_vm_lgkm0<IPH>();
      bare_barrier();
      prep_b(b_more, pb_cur);
      prep_a(a_more, pa_cur);
      hb_dst = half_ptr(ha);
      ha_dst = half_ptr(hb);
      const int ha1 = hb + 1 == NH ? 0 : hb + 1;  // tile t+1's halves
      const int hb1 = ha1 + 1 == NH ? 0 : ha1 + 1;
      const char* pa_n = half_ptr(ha1);  // (after the last tile: slots nobody reads; in bounds)
      const char* pb_n = half_ptr(hb1);
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        mfma_pair(1, p);
        if (p % 2) lb.load_one(pb_cur, p / 2, hb_dst);
        frag_read(pa_n, pb_n, 0, 0, p);
        __builtin_amdgcn_sched_barrier(0);
      }
      ha = ha1;
    }
    wait_vmcnt<0>();  // no zero-fill DMA may land in the staged epilogue's LDS
  }
  if constexpr (STAGED) {
    static_assert(w4_staged_epi(EPI), "staged epilogue: bf16 outputs");
    __bf16* lds = reinterpret_cast<__bf16*>(smem);
    if constexpr (BMODE == B_DUAL)
      w4_epilogue_staged_dual<EPI>(args, acc, m0, n0, lane, wm, wn, lds);
    else  // (STORE_BF16 is launched staged at beta = 0 only)
      w4_epilogue_staged<EPI>(args, acc, m0, n0, lane, wm, wn, lds);
  } else {
    w4_epilogue_direct<BMODE, EPI>(args, acc, m0, n0, lane, wm, wn);
  }
}

}  // namespace fgemm
