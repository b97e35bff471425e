// pa_latent.hip — the LATENT cache layout on gfx950 matrix cores.
//
// Replaces the reference's latent route (kv_cache_layout = "LATENT", attention.rs:4058-4062,
// :4210-4213): one kv-head whose key rows of D dims (e.g. 576 = 512 latent + 64 rotary dims) are
// also the value rows, values being their first VD dims; every query head attends the same rows.
//
// Work unit: one workgroup of 4 wavefronts per (sequence, block of 16 NG grouped query rows,
// context chunk): NG = 2 row groups once a sequence has 32 or more rows, so a row is read once for
// 32 heads.  Rows r = (query token r / H, head r % H), MFMA column c of group j = row row0 + 16 j +
// c.  The
// four wavefronts split the head dims instead of the rows: wavefront w
//   - computes the partial scores of its quarter of the k-steps (dims 32 s .. 32 s + 31 for
//     s in [KS w / 4, KS (w + 1) / 4), KS = D / 32) with 16x16x32 MFMAs, K tile x Q^T;
//   - adds the four partial score tiles read back from LDS (one barrier per step, two buffers),
//     in the same order in every wavefront, so all four hold the same scores and run the same
//     online softmax;
//   - accumulates P . V for its quarter of the value dims (VD / 4 columns), P split into hi + lo
//     16-bit parts, from value-row slices of the step's rows.
// Paged steps (block size a multiple of 16, every row in the pages, rows of at most 576 dims) go
// through a three-slot LDS ring: each 32-row step is copied to LDS by direct loads of whole
// 128-byte lines, every slot but the one being read in flight, and both the key operands and
// the value-row slices are read from there, so every row byte leaves HBM once per workgroup;
// the step's one barrier (the partial-score exchange) also publishes the next step.  Other steps (new rows from the batch, other block sizes, longer rows)
// use a three-slot register ring loaded straight from the rows (key pieces of 64 bytes per row
// and instruction, the value slices read a second time: L2 hits).  Partials of split chunks go
// to the workspace at row (token * H + head) * max_splits + split (stride D), merged by
// split_reduce_kernel as the VALU kernel's are.  The chunk length comes from the host's
// per-sequence lengths when the caller gives them (pa_api.cpp, latent_chunk).
#include "pa_tiles.hpp"

namespace pa {
namespace {

constexpr int kLatMaxKs = 20;  // k-steps of 32 dims in a key row: D <= 640

#ifndef PA_LATENT_DEPTH
#define PA_LATENT_DEPTH 3  // register ring slots: steps loaded DEPTH - 1 ahead of the compute
#endif
#ifndef PA_LATENT_LDS
#define PA_LATENT_LDS 1  // paged steps staged in LDS by direct loads (else the register ring)
#endif
#ifndef PA_LATENT_LDS_SLOTS1
#define PA_LATENT_LDS_SLOTS1 3
#endif
// LDS ring of paged steps: slots of 32 rows x D / 8 16-byte pieces for D <= 576 (the MLA
// 576-dim rows), three of them (124 KiB of LDS with one row group's partial-score buffer, 140
// KiB with two).  Four slots with one row group (exactly the 160 KiB) measured the same once
// every slot prefetches (16-head step 118.4 against 117.9 us).  Longer rows take the register
// ring.
constexpr int kLatLdsMaxD = 576;
constexpr int kLatSlotChunks = 32 * kLatLdsMaxD / 8;
template <int NG>
constexpr int lat_lds_slots() {
  return NG == 1 ? PA_LATENT_LDS_SLOTS1 : 3;
}

// One direct LDS load: 16 bytes per lane from src to LDS byte address lds + 16 * lane.  Written
// as inline assembly so that the compiler's memory-counter bookkeeping does not see it: the
// builtin form made every later LDS read and barrier wait for all outstanding direct loads (the
// prefetched steps included).  The kernel waits for these loads itself (lat_wait_vm) before the
// barrier that publishes a step.
// M0 (the LDS base of the load) is a reserved register: the compiler sets it before each
// instruction of its own that reads it and this kernel has none, so the clobber is declared for
// the record and its warning silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lat_dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most n of this wavefront's vector-memory operations are outstanding (n is
// wave-uniform; the s_waitcnt immediate must be a constant).  Encoding: vmcnt in bits 3:0 and
// 15:14, expcnt (7) and lgkmcnt (15) left at their maxima.
__device__ __forceinline__ void lat_wait_vm(int n) {
#define LAT_VM(k) \
  case k:         \
    __builtin_amdgcn_s_waitcnt(((k) & 15) | (((k) >> 4) << 14) | 0x0F70); \
    break;
  switch (n) {
    LAT_VM(1) LAT_VM(2) LAT_VM(3) LAT_VM(4) LAT_VM(5) LAT_VM(6) LAT_VM(7) LAT_VM(8) LAT_VM(9)
    LAT_VM(10) LAT_VM(11) LAT_VM(12) LAT_VM(13) LAT_VM(14) LAT_VM(15) LAT_VM(16) LAT_VM(17)
    LAT_VM(18) LAT_VM(19) LAT_VM(20) LAT_VM(21) LAT_VM(22) LAT_VM(23) LAT_VM(24) LAT_VM(25)
    LAT_VM(26) LAT_VM(27) LAT_VM(28) LAT_VM(29) LAT_VM(30)
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
#undef LAT_VM
}

// Piece x of row r of an LDS step slot sits at position x ^ (r & 7) within the row's leading
// multiple of 8 pieces: the 16 rows an MFMA operand read touches spread over the banks.
__device__ __forceinline__ int lat_swz(int x, int r, int cpr8) { return x < cpr8 ? x ^ (r & 7) : x; }

template <int DW>
__device__ __forceinline__ VRow<DW> lat_lds_vrow(const char* p) {
  VRow<DW> v;
  __builtin_memcpy(&v, p, sizeof(v));
  return v;
}

// Value operand of N-tile j (8 keys x head dim (DW/16) c + j) from the eight value-row slices
// of a step, as value_operand does for a Step.
template <typename TT, int DW>
__device__ __forceinline__ typename TT::vec8 lat_value_operand(const VRow<DW> (&v)[8], int j) {
  u32x4 w;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t lo = v[2 * m].word(j >> 1), hi = v[2 * m + 1].word(j >> 1);
    w[m] = __builtin_amdgcn_perm(hi, lo, (j & 1) ? 0x07060302u : 0x05040100u);
  }
  return __builtin_bit_cast(typename TT::vec8, w);
}

template <int DW, int KW>
struct LatStep {
  u32x4 k[2][KW];          // this wavefront's key k-steps of tiles A / B (row c, dims 32 s + 8 G)
  VRow<DW> v[8];          // value rows 4 G + e of tile A (e < 4) and B (e >= 4), its dims
};

// NW wavefronts per workgroup, each with VD / NW value dims (DW).  With the register ring:
// two workgroups per CU at 128 value dims, one from 256 on (the ring of five key k-steps and
// eight value-row slices per slot takes ~300 registers at 256, ~400 at 512).  With the LDS ring
// (LDSK, 120 KiB of steps): one workgroup per CU.  (Eight wavefronts of 64 value dims, two per
// SIMD with the register ring, measured 6 % slower at 512 value dims.)
template <int DW, int NG, int NW, bool LDSK>
constexpr int lat_waves_per_simd() {
  return LDSK ? 1 : (DW > 32 || NG > 1 ? 1 : 2);
}

template <typename TT, int DW, bool CAP, int NG, int NW, bool LDSK>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(
    lat_waves_per_simd<DW, NG, NW, LDSK>(), lat_waves_per_simd<DW, NG, NW, LDSK>()))) void
latent_kernel(const AttnParams p) {
  using vec8 = typename TT::vec8;
  constexpr int DL = DW / 16;  // N-tiles (and value dims per lane) of a wavefront
  constexpr int KW = (kLatMaxKs + NW - 1) / NW;  // k-steps per wavefront, at most
  // partial score tiles: [buffer][wavefront][row group][tile][lane]
  __shared__ f32x4 part[2][NW][NG][2][64];
  // LDS ring of paged steps: slot = 32 rows of D / 8 16-byte pieces (row-major, swizzled)
  constexpr int kLatLdsSlots = lat_lds_slots<NG>();
  __shared__ u32x4 lring[LDSK ? kLatLdsSlots * kLatSlotChunks : 1];
  const int rb = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 15, G = lane >> 4;
  const int D = p.head_dim, KS = D / 32;
  const int ks0 = (KS * wave) / NW, nks = (KS * (wave + 1)) / NW - ks0;
  // Everything up to the step loop is uniform over the workgroup (barriers inside the loop).
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int nq = s1 - s0;
  const int H = p.num_heads;  // one kv-head: g = H rows per query token
  const int R = H * nq;
  const int row0 = rb * 16 * NG;
  if (nq <= 0 || row0 >= R) return;
  const int pastb = clamped_past(p, b, nq);
  const int total = seq_total(p, b, pastb, nq);
  const int start = split * p.chunk;
  if (start >= total) return;
  const int end = min(start + p.chunk, total);
  const bool single = start == 0 && end == total;
  if (!single && p.part_o == nullptr) return;
  const int r_last = min(row0 + 16 * NG, R) - 1;
  const int hi_any = p.causal ? pastb + r_last / H + 1 : total;
  const int lo_any = p.window > 0 ? max(0, pastb + row0 / H - p.window + 1) : 0;
  const int t_first = max(start, (lo_any / 32) * 32);
  const int t_last = min(end, hi_any);
  const int nsteps = t_last > t_first ? (t_last - t_first + 31) / 32 : 0;
  // keys every row of the block sees: steps inside need no position tests
  const int all_hi = min(end, p.causal ? pastb + row0 / H + 1 : total);
  const int all_lo = p.window > 0 ? pastb + r_last / H - p.window + 1 : 0;

  const WaveInfo w = make_wave(p, D, b, 0, s0, pastb, total);
  // This lane's query row in each row group (MFMA column c of group j: row row0 + 16 j + c)
  // and the keys it sees.
  // A negative scale moves its sign into the query operands.
  const uint32_t qxor = p.scale < 0.0f ? 0x80008000u : 0u;
  const float scale = fabsf(p.scale), scale_log2 = fabsf(p.scale_log2);
  const float cap_k = CAP ? scale / p.softcap : 0.0f, cap_l2 = p.softcap * kLog2e;
  // Every wavefront runs KW k-steps: those past its own (k >= nks) read k-step KS - 1
  // again against zero query operands, so the loop carries no branch around loads or MFMAs.
  RowState<TT, DW> rs[NG];
  vec8 qv[NG][KW];
  int kofs[KW];  // byte offset of the lane's 16 bytes of each k-step in a key row
#pragma unroll
  for (int k = 0; k < KW; ++k) kofs[k] = 64 * min(ks0 + k, KS - 1) + 16 * G;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int r = row0 + 16 * j + c;
    const bool rvalid = r < R;
    const int qi = rvalid ? r / H : 0, head = rvalid ? r % H : 0;
    const int rpos = pastb + qi;
    rs[j].vis_lo = p.window > 0 ? rpos - p.window + 1 : 0;
    rs[j].vis_hi = rvalid ? (p.causal ? rpos + 1 : total) : -1;
    rs[j].m_run = kNegInf;
    rs[j].l_part = 0.0f;
#pragma unroll
    for (int n = 0; n < DL; ++n) rs[j].o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    const char* qrow =
        reinterpret_cast<const char*>(p.q) + (((int64_t)(s0 + qi) * H + head) * D) * 2 + 16 * G;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      const u32x4 v = (k < nks && rvalid) ? (ld16(qrow + 64 * (ks0 + k)) ^ qxor)
                                          : u32x4{0u, 0u, 0u, 0u};
      qv[j][k] = __builtin_bit_cast(vec8, v);
    }
  }

  // Page ids of the chunk: one block-table window of 64 entries (the host keeps a chunk within
  // 64 blocks of 16 or more rows).
  PageWindow pw;
  window_at(pw, w, min(div_bs(t_first, w), w.max_blocks - 1), lane);
  const int vcol = 2 * (DW * wave + DL * c);  // byte offset of this lane's value dims in a row
  // The sequence's last row (PAGED steps): value rows past the end read it again, so every value
  // operand is a finite cache row and needs no masking (their probabilities are 0).
  const char* last_row;
  {
    const int bi = min(div_bs(total - 1, w), w.max_blocks - 1);
    int64_t blk = __builtin_amdgcn_readlane(pw.ids, min(max(bi - pw.first, 0), 63));
    blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
    last_row = w.kc + (blk * w.bs + mod_bs(total - 1, w)) * w.rowb;
  }
  // PAGED: 16-key tiles wholly in the pages (block size a multiple of 16, every row of the chunk
  // in the cache): one page id per tile; else row by row (new rows from the batch, other block
  // sizes; rows past the end read the last row).
  auto load = [&](auto PAGED, LatStep<DW, KW>& st, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      const int t = t0 + 16 * T;
      const char* kr;
      const char* vr[4];
      if constexpr (decltype(PAGED)::value) {
        const int bi = min(div_bs(t, w), w.max_blocks - 1);
        int64_t blk = __builtin_amdgcn_readlane(pw.ids, min(max(bi - pw.first, 0), 63));
        blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
        const char* tb = w.kc + (blk * w.bs + mod_bs(t, w)) * w.rowb;
        kr = tb + (int64_t)c * w.rowb;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          vr[e] = t + 4 * G + e < total ? tb + (int64_t)(4 * G + e) * w.rowb : last_row;
      } else {
        kr = row_ptr(w, t + c, false, D);
#pragma unroll
        for (int e = 0; e < 4; ++e) vr[e] = row_ptr(w, t + 4 * G + e, false, D);
      }
#pragma unroll
      for (int k = 0; k < KW; ++k) st.k[T][k] = ld16s(kr + kofs[k]);
#pragma unroll
      for (int e = 0; e < 4; ++e) st.v[4 * T + e] = ld_vrow_s<DW>(vr[e] + vcol);
    }
  };
  // Softmax and P . V of step k from its full score tiles (fa: keys t0 .. t0 + 15, fb: the next
  // 16) and the value-row slices in st.
  auto finish = [&](LatStep<DW, KW>& st, int k, const f32x4 (&fa)[NG], const f32x4 (&fb)[NG]) {
    const int t0 = t_first + 32 * k;
    const bool masked = !(t0 >= all_lo && t0 + 32 <= all_hi);
    vec8 phi[NG], plo[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sv = e < 4 ? fa[j][e & 3] : fb[j][e & 3];
        x[e] = CAP ? softcap_log2(sv, cap_k, cap_l2) : sv * scale_log2;
      }
      if (masked) {
        // positions [vis_lo, min(end, vis_hi)) of the row, one unsigned range test per score
        const int hi_pos = min(end, rs[j].vis_hi);
        const unsigned span =
            hi_pos > rs[j].vis_lo ? (unsigned)hi_pos - (unsigned)rs[j].vis_lo : 0u;
        const unsigned rel = (unsigned)(t0 + 4 * G) - (unsigned)rs[j].vis_lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const unsigned off = 16 * (e >> 2) + (e & 3);
          x[e] = (rel + off < span) ? x[e] : kNegInf;
        }
      }
      float lmax = kNegInf;
#pragma unroll
      for (int e = 0; e < 8; ++e) lmax = fmaxf(lmax, x[e]);
      if (__any(needs_rescale(rs[j], lmax))) rescale_rows(rs[j], lmax, G);
      step_probs<TT, DW, false, false>(rs[j], x, scale_log2, 1.f, 1.f, phi[j], plo[j]);
    }
#pragma unroll
    for (int n = 0; n < DL; ++n) {
      const vec8 vb = lat_value_operand<TT, DW>(st.v, n);
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        rs[j].o[n] = TT::mfma(phi[j], vb, rs[j].o[n]);
        rs[j].o[n] = TT::mfma(plo[j], vb, rs[j].o[n]);
      }
    }
  };
  // Partial scores of this wavefront's k-steps, summed across the wavefronts through LDS.
  // mid(): between the partial-score writes and their reads -- the workgroup barrier, with
  // whatever the caller's ring does at it.
  auto compute = [&](LatStep<DW, KW>& st, int k, auto&& mid) {
    const int buf = k & 1;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KW; ++kk) {
        if (kk < nks) {
          sa = TT::mfma(__builtin_bit_cast(vec8, st.k[0][kk]), qv[j][kk], sa);
          sb = TT::mfma(__builtin_bit_cast(vec8, st.k[1][kk]), qv[j][kk], sb);
        }
      }
      part[buf][wave][j][0][lane] = sa;
      part[buf][wave][j][1][lane] = sb;
    }
    mid();
    f32x4 fa[NG], fb[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      fa[j] = part[buf][0][j][0][lane];
      fb[j] = part[buf][0][j][1][lane];
#pragma unroll
      for (int u = 1; u < NW; ++u) {
        fa[j] += part[buf][u][j][0][lane];
        fb[j] += part[buf][u][j][1][lane];
      }
    }
    finish(st, k, fa, fb);
  };

  // Three-slot ring: the rows of step k + 2 are issued before step k is computed.  Every slot
  // is loaded unconditionally (steps past the last one read the last step again, in bounds), so
  // the loads carry no branch and the compiler's memory-counter waits stay exact: a load
  // skipped on one path made it wait for every outstanding load, the prefetch included.
  auto steps = [&](auto PAGED) __attribute__((always_inline)) {
    constexpr int DEPTH = PA_LATENT_DEPTH;
    LatStep<DW, KW> st[DEPTH];
    const int last = t_first + 32 * (nsteps - 1);
    auto at = [&](int k) { return min(t_first + 32 * k, last); };
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i) load(PAGED, st[i], at(i));
    for (int k = 0; k < nsteps; k += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        load(PAGED, st[(i + DEPTH - 1) % DEPTH], at(k + i + DEPTH - 1));
        if (i == 0 || k + i < nsteps) compute(st[i], k + i, [] { __syncthreads(); });
      }
    }
  };
  // LDS-staged paged steps.  Each 32-row step goes to an LDS slot by direct loads (16 bytes per
  // lane, whole 128-byte lines of the page rows per instruction): wavefront w fetches pieces
  // [w D, (w + 1) D) of the slot's 4 D, i.e. ceil(D / 64) loads per step.  The operands are then
  // read from LDS in the register-ring layout (keys: row c of a tile, k-step pieces; values: the
  // wavefront's value-dim slice of eight rows) and computed as there.  Steps are issued two
  // ahead; before step k each wavefront waits for its own loads of step k (the count of its
  // later loads still allowed outstanding), then the workgroup barrier makes every wavefront's
  // pieces visible and frees the slot of step k - 1 for step k + 2.
  auto lds_steps = [&]() __attribute__((always_inline)) {
    const int CPR = D / 8, CPR8 = CPR & ~7;
    const int NIW = (D + 63) / 64;  // direct loads per wavefront and step (D % 64 is 0 or 32)
    int pk[kLatMaxKs / 2];          // per load: (row offset in its page + piece offset) << 5 | row
#pragma unroll
    for (int i = 0; i < kLatMaxKs / 2; ++i) {
      const int s = wave * D + 64 * i + lane;
      const int r = min(s / CPR, 31), xp = s - (s / CPR) * CPR;
      pk[i] = (((r & 15) * (int)w.rowb + 16 * lat_swz(xp, r, CPR8)) << 5) | r;
    }
    // the same plan split for the common case: offsets, and a bit per load for rows 16..31
    int poff[kLatMaxKs / 2];
    uint32_t hi16 = 0;
#pragma unroll
    for (int i = 0; i < kLatMaxKs / 2; ++i) {
      poff[i] = pk[i] >> 5;
      hi16 |= (uint32_t)((pk[i] & 31) >= 16) << i;
    }
    char* const lbase = reinterpret_cast<char*>(&lring[0]);
    // LDS byte address of the ring (the address-space-3 pointer's value)
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lbase;
    // Page cursor of the next step to issue (steps are issued once each, in order): block-table
    // index and row in the block of its first key, advanced by 32 keys per step.
    int cur_bi = div_bs(t_first, w), cur_ob = mod_bs(t_first, w);
    auto issue = [&](int k) __attribute__((always_inline)) {
      const int t0 = t_first + 32 * k;
      const char* tb[2];
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        int bi = cur_bi, ob = cur_ob + 16 * T;
        if (ob >= w.bs) {  // the block size is a multiple of 16
          ob -= w.bs;
          ++bi;
        }
        bi = min(bi, w.max_blocks - 1);
        int64_t blk = __builtin_amdgcn_readlane(pw.ids, min(max(bi - pw.first, 0), 63));
        blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
        tb[T] = w.kc + (blk * w.bs + ob) * w.rowb;
      }
      cur_ob += 32;
      while (cur_ob >= w.bs) {  // at most twice (block size >= 16)
        cur_ob -= w.bs;
        ++cur_bi;
      }
      const uint32_t ldst = __builtin_amdgcn_readfirstlane(
          lds0 + (k % kLatLdsSlots) * (kLatSlotChunks * 16) + wave * D * 16);
      if (D % 64 == 0 && t0 + 32 <= total) {
        // every lane loads, every row of the step is a sequence row
#pragma unroll
        for (int i = 0; i < kLatMaxKs / 2; ++i) {
          if (i < NIW) {
            const char* src = ((hi16 >> i) & 1u ? tb[1] : tb[0]) + poff[i];
            lat_dma16(src, ldst + 1024 * i);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < kLatMaxKs / 2; ++i) {
          if (i < NIW && 64 * i + lane < D) {
            const int r = pk[i] & 31, off = pk[i] >> 5;
            // rows past the sequence end read the last row (finite values under probability 0)
            const char* src = t0 + r < total ? (r < 16 ? tb[0] : tb[1]) + off
                                             : last_row + (off - (r & 15) * (int)w.rowb);
            lat_dma16(src, ldst + 1024 * i);
          }
        }
      }
    };
    auto fill = [&](LatStep<DW, KW>& st, int k) __attribute__((always_inline)) {
      const char* const sb = lbase + (k % kLatLdsSlots) * (kLatSlotChunks * 16);
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        const int r = 16 * T + c;
#pragma unroll
        for (int kk = 0; kk < KW; ++kk) {
          const int x = 4 * min(ks0 + kk, KS - 1) + G;
          st.k[T][kk] = *reinterpret_cast<const u32x4*>(sb + (r * CPR + lat_swz(x, r, CPR8)) * 16);
        }
      }
      const int vb = vcol >> 4, vw = vcol & 15;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = 16 * (e >> 2) + 4 * G + (e & 3);
        st.v[e] = lat_lds_vrow<DW>(sb + (r * CPR + lat_swz(vb, r, CPR8)) * 16 + vw);
      }
    };
#pragma unroll
    for (int i = 0; i < kLatLdsSlots; ++i)
      if (i < nsteps) issue(i);
    // One barrier per step: the one between the partial-score writes and reads of step k also
    // publishes step k + 1's pieces (each wavefront waits for its own loads first) and frees
    // the slot step k was read from (its operands are in registers by then) for step k + S.
    auto wait_loads = [&](int later) __attribute__((always_inline)) {
      // 576-dim rows in the steady state (four or three slots): no search for the immediate
      if (NIW == 9 && later == 18)
        __builtin_amdgcn_s_waitcnt((18 & 15) | ((18 >> 4) << 14) | 0x0F70);
      else if (NIW == 9 && later == 9)
        __builtin_amdgcn_s_waitcnt(9 | 0x0F70);
      else
        lat_wait_vm(later);
    };
    wait_loads(min(kLatLdsSlots - 1, nsteps - 1) * NIW);  // loads issued after step 0's
    __syncthreads();
    auto next = [&](int k) __attribute__((always_inline)) {
      if (k + 1 < nsteps) wait_loads(min(kLatLdsSlots - 2, nsteps - 2 - k) * NIW);
      __syncthreads();
      if (k + kLatLdsSlots < nsteps) issue(k + kLatLdsSlots);
    };
    for (int k = 0; k < nsteps; ++k) {
      LatStep<DW, KW> st;
      fill(st, k);
      compute(st, k, [&] { next(k); });
    }
  };
  // every row the steps read below the sequence end in the pages, pages of whole 16-key tiles,
  // one window of page ids (rows past the end are zeroed or masked)
  if (nsteps <= 0) {
  } else if (w.bs % 16 == 0 && w.cache_limit >= min(w.total, t_first + 32 * nsteps) &&
             div_bs(t_first + 32 * nsteps - 1, w) - pw.first < 64 && (!LDSK || D <= kLatLdsMaxD)) {
    if constexpr (LDSK)
      lds_steps();
    else
      steps(std::true_type{});
  } else {
    steps(std::false_type{});
  }

  // Rows 4 G + i of this lane's O registers in each group: this wavefront's DW value dims.
  const int VD = NW * DW;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    float l_row = rs[j].l_part + __shfl_xor(rs[j].l_part, 16, 64);
    l_row += __shfl_xor(l_row, 32, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + 16 * j + 4 * G + i;
      const float mi = __shfl(rs[j].m_run, 4 * G + i, 64);
      const float li = __shfl(l_row, 4 * G + i, 64);
      if (rr >= R) continue;
      const int oh = rr % H;
      const int64_t t = s0 + rr / H;
      if (single) {
        const float f = finalize_factor(mi, li, sink_logit<TT>(p, oh));
        typename TT::raw vals[DL];
#pragma unroll
        for (int n = 0; n < DL; ++n) vals[n] = TT::from_f32(rs[j].o[n][i] * f);
        typename TT::raw* dst = reinterpret_cast<typename TT::raw*>(p.out) +
                                (t * H + oh) * VD + DW * wave + DL * c;
        if constexpr (DL == 8) {
          u32x4 pk;
#pragma unroll
          for (int m = 0; m < 4; ++m)
            pk[m] = (uint32_t)vals[2 * m] | ((uint32_t)vals[2 * m + 1] << 16);
          *reinterpret_cast<u32x4*>(dst) = pk;
        } else {
#pragma unroll
          for (int n = 0; n < DL; ++n) dst[n] = vals[n];
        }
      } else {
        const int64_t pi = (t * H + oh) * p.max_splits + split;
        float* dst = p.part_o + pi * D + DW * wave + DL * c;
#pragma unroll
        for (int n = 0; n < DL; ++n) dst[n] = rs[j].o[n][i];
        if (wave == 0 && c == 0) {
          p.part_ml[pi * 2 + 0] = mi;
          p.part_ml[pi * 2 + 1] = li;
        }
      }
    }
  }
}

template <typename TT, int DW, int NW>
void launch_lat_dw(const AttnParams& p, dim3 grid, int ng, hipStream_t s) {
  const dim3 block(64 * NW);
  if (ng == 2) {
    if (p.softcap > 0.0f)
      hipLaunchKernelGGL((latent_kernel<TT, DW, true, 2, NW, PA_LATENT_LDS != 0>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((latent_kernel<TT, DW, false, 2, NW, PA_LATENT_LDS != 0>), grid, block, 0, s, p);
  } else if (p.softcap > 0.0f) {
    hipLaunchKernelGGL((latent_kernel<TT, DW, true, 1, NW, PA_LATENT_LDS != 0>), grid, block, 0, s, p);
  } else {
    hipLaunchKernelGGL((latent_kernel<TT, DW, false, 1, NW, PA_LATENT_LDS != 0>), grid, block, 0, s, p);
  }
}

template <typename TT>
void launch_lat_t(const AttnParams& p, dim3 grid, int ng, hipStream_t s) {
  switch (p.v_head_dim) {
    case 128: launch_lat_dw<TT, 32, 4>(p, grid, ng, s); break;
    case 256: launch_lat_dw<TT, 64, 4>(p, grid, ng, s); break;
    default: launch_lat_dw<TT, 128, 4>(p, grid, ng, s); break;
  }
}

}  // namespace

// Key rows of D = 32 k dims up to 640, values = their first 128, 256 or 512 dims, 16-bit
// activations with the cache in the same type.
bool latent_mfma_supported(int head_dim, int v_head_dim, pa_dtype act, pa_dtype cache_dtype) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (cache_dtype != act) return false;
  if (head_dim % 32 != 0 || head_dim > 32 * kLatMaxKs) return false;
  return (v_head_dim == 128 || v_head_dim == 256 || v_head_dim == 512) && v_head_dim <= head_dim;
}

// Grid: one workgroup per (16 grouped query rows, context chunk, sequence).
hipError_t launch_latent(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype, hipStream_t s) {
  if (!latent_mfma_supported(p.head_dim, p.v_head_dim, act, cache_dtype) || p.kv_heads != 1 ||
      !p.v_from_key)
    return hipErrorInvalidValue;
  if (p.batch <= 0 || p.num_tokens <= 0) return hipSuccess;
  if (p.chunk < 32 || p.chunk % 32 != 0 || p.max_splits < 1 || p.max_splits > 65535 ||
      p.batch > 65535)
    return hipErrorInvalidValue;
  const int mq = p.max_query_len > 0 ? p.max_query_len : p.num_tokens;
  const int ng = latent_row_groups(p.num_heads, mq);
  const int64_t rbs = ((int64_t)p.num_heads * mq + 16 * ng - 1) / (16 * ng);
  if (rbs > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((unsigned)rbs, p.max_splits, p.batch);
  if (act == PA_DTYPE_FLOAT16)
    launch_lat_t<TF16>(p, grid, ng, s);
  else
    launch_lat_t<TBF16>(p, grid, ng, s);
  return hipGetLastError();
}

}  // namespace pa
