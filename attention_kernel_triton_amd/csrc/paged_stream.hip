// Stream-K paged var-len decode for gfx950 (the automatic-chunk path of
// decode_flash_attention_redundant_var_len_paged.py:70-224).
//
// Work decomposition.  A "unit" is one (sequence b, head group y): the up to
// GT query heads of one kv head that read the same K/V rows.  Every unit's
// K/V is cut into 16-token groups (a page of page_size tokens holds
// page_size / 16 of them), and the groups of all units are laid out on one
// axis, kv-head-group major:
//   g = y * TG + position * gpp + slice,   TG = total_pages * gpp,
// where `position` indexes kv_page_indices, so sequence b's groups of head
// group y are the contiguous range [y*TG + indptr[b]*gpp, y*TG + indptr[b+1]*gpp).
// The W waves of the launch take equal contiguous ranges of that axis
// (wave w: [w*N/W, (w+1)*N/W)), fixed before the launch: no tickets, no
// workgroup barriers after the prologue.  A wave streams its range with two
// groups in flight, keeps one online softmax for the unit it is in, and at
// each unit boundary either writes the unit's output (a unit wholly inside
// the wave) or stores a partial (m, l, o).  Only a wave's first and last
// segments can be partial.  At its end a wave counts its partials in their
// units' arrival counters; the wave that counts a unit's last partial merges
// them (log-sum-exp over the contiguous waves that cover the unit, in wave
// order, so results do not depend on timing) and writes the output.
//
// Per group: four (D=128) v_mfma_f32_16x16x32_f16 give the 16-token x 16-head
// score block as S^T (lane (R, c) holds head c, tokens 4R .. 4R+3); the online
// softmax runs in log2 units; P is rounded to fp16 as the reference rounds it
// (decode_flash_attention_redundant_var_len_paged.py:186); P.V is D/16
// v_mfma_f32_16x16x16_f16 with P^T straight from the score lanes and V^T read
// from an LDS copy of the group's V rows with ds_read_b64_tr_b16.
#include <math.h>

#include "akt_common.hpp"
#include "akt_host.hpp"
#include "paged_stream.hpp"

namespace akt {
namespace {

#define AKT_SNEG_INF (-__builtin_inff())

// Last index i in [0, n] with s[i] <= x, given a non-decreasing s[0..n];
// -1 if s[0] > x.
__device__ __forceinline__ int last_le(const int* s, int n, int x) {
  int lo = 0, hi = n + 1;  // first index with s > x lies in [lo, hi]
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (s[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo - 1;
}

// Waves per SIMD the instance is built for: two up to D = 128 (at most ~180
// VGPRs whatever the head count: P.V accumulates in D/4 registers), one at
// D = 256.
template <int D, int GT>
constexpr int stream_min_waves() {
  return D <= 128 ? 2 : 1;
}
// Threads per workgroup: with two waves per SIMD, one 512-thread workgroup per
// CU, so that the two waves sharing a SIMD (waves w and w + 4) are in one
// workgroup and can see each other's progress; otherwise 256.
template <int D, int GT>
constexpr int stream_threads() {
  return stream_min_waves<D, GT>() == 2 ? 512 : 256;
}

// Groups in flight per wave: after a group is consumed, the group PD ahead is
// issued into its buffer.  (Three measured slower on config 3.)
template <int D, int GT>
constexpr int stream_depth() {
  return 2;
}

template <int D, int GT>
__global__ __launch_bounds__((stream_threads<D, GT>()))
__attribute__((amdgpu_waves_per_eu(stream_min_waves<D, GT>(), 8))) void paged_stream_kernel(
    StreamParams p) {
  constexpr int PD = stream_depth<D, GT>();
  constexpr int kSThreads = stream_threads<D, GT>();
  constexpr int kSWaves = kSThreads / kWave;
  constexpr bool PAIRED = kSWaves == 8;
  constexpr int KS = D / 32;                 // MFMA k-steps (8 elements each)
  constexpr int VTOK = (D == 64) ? 2 : 4;    // V tokens per lane per group
  constexpr int VDIM = (D == 256) ? 16 : 8;  // V dims per lane
  constexpr int VLD = VDIM / 8;              // 16-byte loads per V token
  constexpr int NT = D / 16;                 // 16-dim output tiles (P.V MFMAs per group)
  constexpr int VROW = D + 16;               // staged V row (fp16): padded against bank conflicts

  // Sequence page ranges: sequence b owns positions [sm_s[b], sm_s[b + 1]) of
  // kv_page_indices (indptr clamped to [0, total_pages] and made
  // non-decreasing).
  __shared__ int sm_s[kStreamMaxBatch + 1];
  __shared__ int sm_wmax[kSWaves];
  // Groups each wave has consumed (paired waves only).
  __shared__ int sm_prog[kSWaves];
  // Each wave stages a group's V rows here for the transposing reads of P.V.
  __shared__ __attribute__((aligned(16))) half_t sm_v[kSWaves][16 * VROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int R = lane >> 4;
  const int c16 = lane & 15;
  const uint32_t kOnes = 0x3c003c00u;  // half2(1, 1)
  const int gw = (int)blockIdx.x * kSWaves + wave;
  const int W = p.W;
  const int N = p.N;
  // Wave w's range starts at floor(w N / W): no range is empty while W <= N.
  // With more waves than groups, waves 0 .. N - 1 take one group each and the
  // rest none, so that no empty wave lies inside a unit's run of waves (every
  // wave of that run stores a partial and counts it).
  auto wstart = [&](int w) __attribute__((always_inline)) -> int {
    return W <= N ? (int)(((int64_t)w * N) / W) : min(w, N);
  };
  const int g0 = wstart(gw);
  const int n = wstart(gw + 1) - g0;  // groups of this wave

  // Axis position of group g: head group y, page position pp, 16-row slice.
  auto locate = [&](int g, int& y, int& pp, int& slice) __attribute__((always_inline)) {
    y = g / p.TG;
    const int pos = g - y * p.TG;
    pp = pos / p.gpp;
    slice = pos - pp * p.gpp;
  };
  // ---- lookahead ------------------------------------------------------------
  // The group PD ahead of the one being issued is "fetched": its page id and
  // its sequence's last-page length are read with one vector load each (a
  // uniform address), the same two loads for every group.  (A scalar load
  // would be counted with the LDS accesses and, since scalar loads complete
  // out of order, every LDS wait would then wait for it.)  Its position is
  // tracked in scalar registers, advanced one group per fetch: head group
  // la_y, page position la_pp, 16-row slice la_slice, and sequence la_b
  // (-1 before sequence 0's pages, B past the last) with la_end, the first
  // position past la_b's pages (la_b and la_end need the sequence table).
  // (Sized to the tensors: a read past them returns 0 and touches no memory.)
  const auto idx_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)p.indices, 0,
                                                          p.total_pages * 4, kBufferWord3);
  const auto ll_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)p.last_len, 0, p.B * 4,
                                                         kBufferWord3);
  int la_y = 0, la_pp = 0, la_slice = 0, la_b = -1, la_end = 0;
  auto seq_end = [&](int b) __attribute__((always_inline)) -> int {
    return b < p.B ? uniform(sm_s[b + 1]) : INT32_MAX;
  };
  // One group forward; `track`: keep la_b / la_end (the table exists).
  auto advance = [&](bool track) __attribute__((always_inline)) {
    if (++la_slice < p.gpp) return;
    la_slice = 0;
    if (++la_pp == p.total_pages) {
      la_pp = 0;
      ++la_y;
      la_b = -1;
      if (track) la_end = uniform(sm_s[0]);
    }
    if (track)
      while (la_b < p.B && la_pp >= la_end) la_end = seq_end(++la_b);
  };
  // Sequence of position pp from the table (the last b with start <= pp).
  auto seek = [&](int pp) __attribute__((always_inline)) {
    la_b = uniform(last_le(sm_s, p.B, pp));
    la_end = la_b < 0 ? uniform(sm_s[0]) : seq_end(la_b);
  };
  // A fetched group: page id and last-page length (vector registers, loaded),
  // and its position (wave-uniform).
  struct Fetch {
    int page, ll;
    int b, y, slot, last;
  };
  auto fetch = [&](Fetch& f) __attribute__((always_inline)) {
    f.page = __builtin_amdgcn_raw_buffer_load_b32(idx_rsrc, (uint32_t)la_pp * 4u, 0, 0);
    const bool seq_ok = la_b >= 0 && la_b < p.B;
    const int lb = min(max(la_b, 0), p.B - 1);
    f.ll = __builtin_amdgcn_raw_buffer_load_b32(ll_rsrc, (uint32_t)lb * 4u, 0, 0);
    f.b = seq_ok ? la_b : -1;
    f.y = la_y;
    f.slot = la_slice * 16;
    f.last = seq_ok && la_pp == la_end - 1;
    advance(true);
  };

  // ---- per-lane load offsets ------------------------------------------------
  // A group is the 16 rows from row `slot` of one page: its addresses are a
  // uniform base plus this lane's K row (c16) and K dims (8R + 32s for MFMA
  // k-step s, so that the four lanes of a row read 64 contiguous bytes per
  // load), and its V token tt0 + i at dims dim0.  Groups without a valid page
  // read the q tensor's first row instead (always mapped), inside that row.
  const int dim0 = (D == 64) ? 8 * (c16 & 7) : VDIM * c16;
  const int tt0 = (D == 64) ? (4 * R + 2 * (c16 >> 3)) : 4 * R;
  const uint32_t lane_kofs = (uint32_t)(c16 * p.k_sb + 8 * R) * 2u;
  const uint32_t lane_qofs = (uint32_t)(8 * R) * 2u;
  const uint32_t lane_v0ofs = (uint32_t)(tt0 * p.v_sb + dim0) * 2u;
  const uint32_t lane_dofs = (uint32_t)dim0 * 2u;
  const uint32_t vstep = (uint32_t)p.v_sb * 2u;

  struct Buf {
    uint4_t k[KS];
    uint4_t v[VTOK][VLD];
    half8_t q[KS];  // the query fragment of the group's unit
    // wave-uniform: sequence (-1: none or a dummy), head group, first row of
    // the slice, whether the page is the sequence's last, valid page id,
    // usable tokens
    int b, y, slot, last, use, nv;
  };
  // Usable tokens of a buffer's group given its sequence's last-page length
  // ll (a loaded register): 16, or on the sequence's last page the rows below
  // ll (clamped to [0, page_size]), 0 for invalid pages.  The length is read
  // into a scalar here, when the group is issued (its load, PD groups back,
  // is complete then), so that no vector register holding a loaded value is
  // carried from one group to the next: the compiler may copy such a register
  // at the loop's head, and would wait there for the load that last wrote it.
  auto set_usable = [&](Buf& bf, int ll_reg) __attribute__((always_inline)) {
    const int ll = min(max(uniform(ll_reg), 0), p.page_size);
    const int tail = min(max(ll - bf.slot, 0), 16);
    bf.nv = (!bf.use || bf.b < 0) ? 0 : (bf.last ? tail : 16);
  };

  // Query fragment of unit (b, y) (MFMA B operand): head hq0 + c16, dims
  // 32s + 8R + e (the K loads' assignment).  Columns past the unit's heads
  // repeat head hq0: each column's scores, softmax and P.V stay in that
  // column's lanes, and those lanes store nothing.  (Zeroing them would make
  // the compiler wait for the loads right where they are issued.)  b < 0 (no
  // unit) reads sequence 0's rows, so that every group issues the same loads.
  auto load_q = [&](int b, int y, half8_t (&qd)[KS]) __attribute__((always_inline)) {
    b = max(b, 0);
    const int kvh = p.n_hg == 1 ? y : y / p.n_hg;
    const int hg = y - kvh * p.n_hg;
    const int hq0 = kvh * p.G + hg * GT;
    const int nh = min(GT, p.G - hg * GT);
    const half_t* qrow =
        p.q + (int64_t)b * p.q_sb + (int64_t)(hq0 + (c16 < nh ? c16 : 0)) * p.q_sh + 8 * R;
#pragma unroll
    for (int s = 0; s < KS; ++s) qd[s] = as_half8(ld16(qrow + 32 * s));
  };

  // Issues group j of this wave from its fetch record f (j >= n: a dummy
  // group that reads the q row), then fetches group j + PD into f.
  // `take_ll`: the usable tokens are set from f's last-page length (the
  // prologue sets them itself).  Rows of a
  // valid page are loaded whole; tokens past the usable prefix are masked when
  // consumed.  `seq`: the sequence is known (the table exists), so the unit's
  // q fragment is loaded with the group.  Every call issues the same loads
  // whatever the data: a load issued only on some paths would leave the
  // compiler unsure how many loads follow a buffer's, and it would then wait
  // for all of them before consuming it.
  Fetch fr[PD];
  auto issue = [&](int j, Buf& bf, bool seq, Fetch& f, bool take_ll)
                   __attribute__((always_inline)) {
    const int page = uniform(f.page);
    const int y = f.y, slot = f.slot;
    bf.b = j < n ? f.b : -1;
    bf.y = y;
    bf.slot = slot;
    bf.last = f.last;
    const bool use = j < n && page >= 0 && page < p.num_pool_pages;
    bf.use = use;
    if (take_ll) set_usable(bf, f.ll);
    if (seq) fetch(f);
    if (seq) load_q(bf.b, y, bf.q);
    const int kvh = p.n_hg == 1 ? y : y / p.n_hg;
    const char* kg = reinterpret_cast<const char*>(
        use ? p.kbase + (int64_t)kvh * p.k_head + (int64_t)page * p.k_sa + (int64_t)slot * p.k_sb
            : p.q);
    const uint32_t ko = use ? lane_kofs : lane_qofs;
#pragma unroll
    for (int s = 0; s < KS; ++s) bf.k[s] = ld16(kg + ko + 64 * s);
    const char* vg = reinterpret_cast<const char*>(
        use ? p.vbase + (int64_t)kvh * p.v_head + (int64_t)page * p.v_sa + (int64_t)slot * p.v_sb
            : p.q);
#pragma unroll
    for (int i = 0; i < VTOK; ++i) {
      const uint32_t vo = use ? lane_v0ofs + (uint32_t)i * vstep : lane_dofs;
#pragma unroll
      for (int jj = 0; jj < VLD; ++jj) bf.v[i][jj] = ld16(vg + vo + 16 * jj);
    }
  };

  // ---- prologue ----------------------------------------------------------------
  // The first PD groups' page ids, then group 0's K and V, need only the
  // kernel arguments: they go out before the sequence table is built (its
  // barriers wait for LDS only).  The table gives the groups' sequences, hence
  // their q fragments and last-page lengths.
  if (PAIRED && lane == 0)
    __hip_atomic_store(&sm_prog[wave], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  int y0 = 0, pp0 = 0, slice0 = 0;
  if (n > 0) locate(g0, y0, pp0, slice0);
  la_y = y0;
  la_pp = pp0;
  la_slice = slice0;
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    fr[i].page = __builtin_amdgcn_raw_buffer_load_b32(idx_rsrc, (uint32_t)la_pp * 4u, 0, 0);
    fr[i].y = la_y;
    fr[i].slot = la_slice * 16;
    fr[i].b = -1;
    fr[i].last = 0;
    fr[i].ll = 0;
    advance(false);
  }
  constexpr int ENT = (kStreamMaxBatch + 1 + kSThreads - 1) / kSThreads;  // table entries per thread
  int tv[ENT];
#pragma unroll
  for (int j = 0; j < ENT; ++j) {
    const int e = ENT * tid + j;
    tv[j] = e <= p.B ? min(max(p.indptr[e], 0), p.total_pages) : 0;
  }
  Buf bufs[PD];
  if (n > 0) issue(0, bufs[0], false, fr[0], false);
  // Sequence table: indptr clamped to [0, total_pages] and made
  // non-decreasing (a max-scan).
  {
#pragma unroll
    for (int j = 1; j < ENT; ++j) tv[j] = max(tv[j], tv[j - 1]);
    int incl = tv[ENT - 1];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl = max(incl, t);
    }
    if (lane == 63) sm_wmax[wave] = incl;
    __syncthreads();
    int before = 0;
#pragma unroll
    for (int w = 0; w < kSWaves; ++w)
      if (w < wave) before = max(before, sm_wmax[w]);
    const int up = __shfl_up(incl, 1, 64);
    const int excl = lane > 0 ? max(before, up) : before;
#pragma unroll
    for (int j = 0; j < ENT; ++j) {
      const int e = ENT * tid + j;
      if (e <= p.B) sm_s[e] = max(excl, tv[j]);
    }
    __syncthreads();
  }

  // Sequences without pages have no groups: o = 0 and lse = -inf here.
  for (int bb = gw; bb < p.B; bb += W) {
    if (sm_s[bb] != sm_s[bb + 1]) continue;
    half_t* orow = p.o + (int64_t)bb * p.Hq * D;
    for (int i = lane; i < p.Hq * (D / 8); i += 64) st16(orow + 8 * i, uint4_t{0, 0, 0, 0});
    if (p.lse)
      for (int h = lane; h < p.Hq; h += 64) p.lse[(int64_t)bb * p.Hq + h] = AKT_SNEG_INF;
  }
  if (n <= 0) return;  // wave-uniform; no barrier follows

  // Sequences of groups 0 .. PD-1 (their last-page lengths are loaded into
  // pll), then the lookahead from group PD on.  Group 0's q
  // fragment, group PD's fetch, then groups 1 .. PD-1: each buffer's loads in
  // the order of the main loop's, so that the compiler's wait counts at the
  // loop's entry match those of its iterations.
  la_y = y0;
  la_pp = pp0;
  la_slice = slice0;
  seek(pp0);
  int pll[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    const bool seq_ok = la_b >= 0 && la_b < p.B;
    fr[i].b = seq_ok ? la_b : -1;
    fr[i].last = seq_ok && la_pp == la_end - 1;
    const int lb = min(max(la_b, 0), p.B - 1);
    pll[i] = __builtin_amdgcn_raw_buffer_load_b32(ll_rsrc, (uint32_t)lb * 4u, 0, 0);
    advance(true);
  }
  bufs[0].b = fr[0].b;
  bufs[0].last = fr[0].last;
  load_q(bufs[0].b, bufs[0].y, bufs[0].q);
  fetch(fr[0]);
#pragma unroll
  for (int i = 1; i < PD; ++i) issue(i, bufs[i], true, fr[i], false);
#pragma unroll
  for (int i = 0; i < PD; ++i) set_usable(bufs[i], pll[i]);

  // ---- state of the unit being streamed ------------------------------------
  float m_run = AKT_SNEG_INF;  // running max of head c16 (log2 units)
  float l_part = 0.f;          // sum of fp16-rounded P (normalises O)
  float e_part = 0.f;          // sum of fp32 P (the LSE)
  // O^T tiles of P.V: lane (R, c16) holds dims 16t + 4R + r of head c16.
  float4_t acc[NT];
  int cur_b = -1, cur_y = 0;
  // Unit bookkeeping (wave-uniform): unit id y * B + b (the units' order on
  // the axis, so that wave + unit, the partial slot, is unique: a later wave
  // never holds an earlier unit), heads, covering waves.
  int cu_unit = 0, cu_hq0 = 0, cu_nh = 0, cu_wf = 0, cu_nc = 1;
  // Partial segments to count at the end (at most the first and the last).
  int pa_unit = -1, pa_b = 0, pa_hq0 = 0, pa_nh = 0, pa_wf = 0, pa_nc = 0;
  int pb_unit = -1, pb_b = 0, pb_hq0 = 0, pb_nh = 0, pb_wf = 0, pb_nc = 0;

  // The wave whose range holds group g (the last w with wstart(w) <= g).
  auto wave_of = [&](int g) __attribute__((always_inline)) -> int {
    return W <= N ? (int)(((int64_t)(g + 1) * W - 1) / N) : g;
  };

  auto begin_unit = [&](int b, int y) __attribute__((always_inline)) {
    m_run = AKT_SNEG_INF;
    l_part = 0.f;
    e_part = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int kvh = p.n_hg == 1 ? y : y / p.n_hg;
    const int hg = y - kvh * p.n_hg;
    cu_hq0 = kvh * p.G + hg * GT;
    cu_nh = min(GT, p.G - hg * GT);
    cu_unit = y * p.B + b;  // axis order: slot = wave + unit is then unique
    const int s0 = uniform(sm_s[b]), s1 = uniform(sm_s[b + 1]);
    const int first = y * p.TG + s0 * p.gpp;
    const int last = y * p.TG + s1 * p.gpp - 1;
    cu_wf = wave_of(first);
    cu_nc = wave_of(last) - cu_wf + 1;
  };

  // Scores, online softmax and P.V of one loaded group.  Tokens past the
  // usable prefix (rows past the last page's length) get score -inf and
  // their V rows, which may hold anything, are staged as zeros.
  //   S^T = K . Q^T (16 tokens x 16 heads): A = K rows, B = the q fragment;
  //   O^T += V^T . P^T: one v_mfma_f32_16x16x16_f16 per 16 dims, A = V^T read
  //   from the staged rows with ds_read_b64_tr_b16 (lane (R, c) gets tokens
  //   4R .. 4R+3 of dim 16t + c), B = P^T straight from the score lanes
  //   (lane (R, c) holds head c's probabilities of tokens 4R .. 4R+3).
  half_t* const vst = &sm_v[wave][0];
  auto consume = [&](const Buf& bf, int nv) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < VTOK; ++i)
#pragma unroll
      for (int jj = 0; jj < VLD; ++jj)
        *reinterpret_cast<uint4_t*>(vst + (tt0 + i) * VROW + dim0 + 8 * jj) = bf.v[i][jj];
    if (nv < 16) {  // wave-uniform: zero the rows past the usable prefix (LDS is in order)
#pragma unroll
      for (int i = 0; i < VTOK; ++i)
#pragma unroll
        for (int jj = 0; jj < VLD; ++jj)
          if (tt0 + i >= nv)
            *reinterpret_cast<uint4_t*>(vst + (tt0 + i) * VROW + dim0 + 8 * jj) = uint4_t{0, 0, 0, 0};
    }
    float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) sacc = mfma16x16x32(as_half8(bf.k[s]), bf.q[s], sacc);
    float t[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) t[r] = (4 * R + r < nv) ? sacc[r] * p.qk_scale : AKT_SNEG_INF;
    float mt = fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3]));
    mt = rows_max(mt);
    const float m_new = fmaxf(m_run, mt);
    if (__any(m_new > m_run)) {
      const float alpha = (m_new > m_run) ? fast_exp2(m_run - m_new) : 1.0f;
      l_part *= alpha;
      e_part *= alpha;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == AKT_SNEG_INF) ? 0.f : m_run;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(t[r] - m_use);
    const uint32_t p01 = pack_half2(pr[0], pr[1]);
    const uint32_t p23 = pack_half2(pr[2], pr[3]);
    l_part = dot2(p23, kOnes, dot2(p01, kOnes, l_part));
    e_part += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    const half4_t pb = __builtin_bit_cast(half4_t, (uint2){p01, p23});
    // Source lane (R, c) of the transposing read addresses token 4R + c / 4,
    // dims 16t + 4 (c % 4) .. + 3.  All tiles are read before the first MFMA.
    const half_t* vrd = vst + (4 * R + (c16 >> 2)) * VROW + 4 * (c16 & 3);
    half4_t va[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) va[tt] = __builtin_bit_cast(half4_t, ds_read_tr16(vrd + 16 * tt));
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
      acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[tt], pb, acc[tt], 0, 0, 0);
  };

  // Four normalised output values of row `row` at dims d0 .. d0 + 3.
  auto store_o4 = [&](int64_t row, int d0, float4_t O, float inv) __attribute__((always_inline)) {
    half4_t hv;
#pragma unroll
    for (int r = 0; r < 4; ++r) hv[r] = (half_t)(O[r] * inv);
    *reinterpret_cast<half4_t*>(p.o + row * D + d0) = hv;
  };
  auto store_lse = [&](int64_t row, float M, float E) __attribute__((always_inline)) {
    if (p.lse) p.lse[row] = E > 0.f ? (M + log2f(E)) * kLn2 : AKT_SNEG_INF;
  };

  // End of the current unit's segment: wave reduction, then the output (a
  // unit wholly inside this wave) or a partial at slot gw + unit.
  auto flush = [&]() __attribute__((always_inline)) {
    // Lane (R, c16) holds head c16's dims 16t + 4R + r: only the normalisers
    // are summed over the four rows.
    const float l_w = rows_sum(l_part);
    const float e_w = rows_sum(e_part);
    const bool direct = cu_nc == 1;
    const int64_t slot = (int64_t)gw + cu_unit;
    if (c16 < cu_nh) {
      if (direct) {
        const int64_t row = (int64_t)cur_b * p.Hq + cu_hq0 + c16;
        const float inv = l_w > 0.f ? 1.0f / l_w : 0.f;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) store_o4(row, 16 * tt + 4 * R, acc[tt], inv);
        if (R == 0) store_lse(row, m_run, e_w);
      } else {
        const int64_t ph = slot * GT + c16;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
          st16_device(p.part_o, (uint32_t)((ph * D + 16 * tt + 4 * R) * 4), as_uint4f(acc[tt]));
        if (R == 0)
          st16_device(p.part_ml, (uint32_t)(ph * 16), as_uint4f(float4_t{m_run, l_w, e_w, 0.f}));
      }
    }
    // Value selects (a branch between the two sets makes the compiler select
    // between their addresses, on the stack).
    const bool to_a = !direct && pa_unit < 0;
    const bool to_b = !direct && !to_a;
    pa_b = to_a ? cur_b : pa_b;
    pa_hq0 = to_a ? cu_hq0 : pa_hq0;
    pa_nh = to_a ? cu_nh : pa_nh;
    pa_wf = to_a ? cu_wf : pa_wf;
    pa_nc = to_a ? cu_nc : pa_nc;
    pa_unit = to_a ? cu_unit : pa_unit;
    pb_b = to_b ? cur_b : pb_b;
    pb_hq0 = to_b ? cu_hq0 : pb_hq0;
    pb_nh = to_b ? cu_nh : pb_nh;
    pb_wf = to_b ? cu_wf : pb_wf;
    pb_nc = to_b ? cu_nc : pb_nc;
    pb_unit = to_b ? cu_unit : pb_unit;
  };

  // ---- stream the range, PD groups in flight --------------------------------
  {
    // Balance of the two waves of a SIMD: the older one wins issue
    // arbitration, and with equal ranges it would finish ~15% before the
    // younger one (measured on MI355X).  After each group a wave publishes
    // its progress and runs at raised priority while it is behind its partner.
    int done = 0;
    auto balance = [&]() __attribute__((always_inline)) {
      if constexpr (PAIRED) {
        ++done;
        if (lane == 0)
          __hip_atomic_store(&sm_prog[wave], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int other = uniform(__hip_atomic_load(&sm_prog[wave ^ 4], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_WORKGROUP));
        if (done < other) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
    };
    auto step = [&](Buf& bf) __attribute__((always_inline)) {
      if (bf.b != cur_b || bf.y != cur_y) {  // wave-uniform
        if (cur_b >= 0) flush();
        if (bf.b >= 0) begin_unit(bf.b, bf.y);
        cur_b = bf.b;
        cur_y = bf.y;
      }
      if (bf.nv > 0) consume(bf, bf.nv);
      balance();
    };
    // Every iteration issues its loads (groups past the range read the q
    // row), so the loads after each buffer's are always the same ones.
    for (int j = 0; j < n; j += PD) {
#pragma unroll
      for (int i = 0; i < PD; ++i) {
        if (j + i < n) step(bufs[i]);
        issue(j + i + PD, bufs[i], true, fr[i], true);
      }
    }
    if (cur_b >= 0) flush();
    if constexpr (PAIRED) {
      __builtin_amdgcn_s_setprio(0);
      if (lane == 0)  // done: the partner no longer competes with this wave
        __hip_atomic_store(&sm_prog[wave], 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }

  // ---- count the partials; the last arrival merges its unit -----------------
  if (pa_unit < 0) return;
  // Every partial store of this wave (device scope) is complete before any
  // count; the merging wave reads the partials with device-scope loads.
  __builtin_amdgcn_s_waitcnt(0);
  // Merge layout: lane l owns NVL consecutive float4 vectors of the unit's
  // output (vectors l*NVL .. l*NVL + NVL - 1), all of one head (64 is a
  // multiple of GT), so it needs one (m, l, e) row per partial; U partials
  // are loaded per round trip.
  constexpr int NV = GT * D / 4;               // float4 vectors of a unit's output
  constexpr int NVL = NV >= 64 ? NV / 64 : 1;  // per lane
  constexpr int U = 32 / (NVL + 1) > 0 ? 32 / (NVL + 1) : 1;
  // Counts of both partials, issued before either result is awaited.
  int prev_a = 0, prev_b = 0;
  if (lane == 0) {
    prev_a = atomicAdd(&p.arrive[pa_unit], 1);
    if (pb_unit >= 0) prev_b = atomicAdd(&p.arrive[pb_unit], 1);
  }
  const bool last_a = __builtin_amdgcn_readfirstlane(prev_a) == pa_nc - 1;
  const bool last_b = pb_unit >= 0 && __builtin_amdgcn_readfirstlane(prev_b) == pb_nc - 1;
  // The wave that counted a unit's last partial resets its counter and merges
  // the unit's partials in wave order.
  auto merge = [&](int unit, int b, int hq0, int nh, int wf, int nc) __attribute__((always_inline)) {
    if (lane == 0) atomicExch(&p.arrive[unit], 0);
    const int vec0 = (NV < 64 ? min(lane, NV - 1) : lane * NVL);
    const int h = (vec0 * 4) / D;
    const int d0 = vec0 * 4 - h * D;
    float M = AKT_SNEG_INF, L = 0.f, E = 0.f;
    float4_t Acc[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) Acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nc; c0 += U) {
      float4_t ml[U], ov[U][NVL];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = min(c0 + u, nc - 1);
        const int64_t ph = ((int64_t)wf + c + unit) * GT + h;
        ml[u] = as_float4u(ld16_device(p.part_ml, (uint32_t)(ph * 16)));
#pragma unroll
        for (int i = 0; i < NVL; ++i)
          ov[u][i] = as_float4u(ld16_device(p.part_o, (uint32_t)((ph * D + d0 + 4 * i) * 4)));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float m = ml[u][0];
        if (c0 + u >= nc || m == AKT_SNEG_INF) continue;
        if (m > M) {
          const float s = fast_exp2(M - m);  // 0 while M = -inf (Acc, L, E are 0 then)
#pragma unroll
          for (int i = 0; i < NVL; ++i) Acc[i] *= s;
          L *= s;
          E *= s;
          M = m;
        }
        const float f = fast_exp2(m - M);
#pragma unroll
        for (int i = 0; i < NVL; ++i) Acc[i] += f * ov[u][i];
        L += f * ml[u][1];
        E += f * ml[u][2];
      }
    }
    if ((NV >= 64 || lane < NV) && h < nh) {
      const int64_t row = (int64_t)b * p.Hq + hq0 + h;
      const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
      for (int i = 0; i < NVL; ++i) store_o4(row, d0 + 4 * i, Acc[i], inv);
      if (d0 == 0) store_lse(row, M, E);
    }
  };
  if (last_a) merge(pa_unit, pa_b, pa_hq0, pa_nh, pa_wf, pa_nc);
  if (last_b) merge(pb_unit, pb_b, pb_hq0, pb_nh, pb_wf, pb_nc);
}

// Launches instance (D, GT) on the resident workgroups (two per CU at
// D <= 128 with up to 4 heads per unit), at most kStreamMaxWaves waves and no
// more waves than groups.
template <int D, int GT>
int64_t wave_cap_t() {
  constexpr int waves = stream_threads<D, GT>() / kWave;
  const int cap = resident_blocks(paged_stream_kernel<D, GT>, stream_threads<D, GT>());
  if (cap <= 0) return kStreamMaxWaves;
  return (int64_t)cap * waves < kStreamMaxWaves ? (int64_t)cap * waves : kStreamMaxWaves;
}

template <int D>
int64_t wave_cap_gt(int gt) {
  switch (gt) {
    case 1: return wave_cap_t<D, 1>();
    case 2: return wave_cap_t<D, 2>();
    case 4: return wave_cap_t<D, 4>();
    case 8: return wave_cap_t<D, 8>();
    case 16:
      if constexpr (D != 256) return wave_cap_t<D, 16>();
      break;
  }
  return kStreamMaxWaves;
}

template <int D, int GT>
int launch_stream_t(StreamParams p, hipStream_t st) {
  auto kernel = paged_stream_kernel<D, GT>;
  constexpr int threads = stream_threads<D, GT>();
  constexpr int waves = threads / kWave;
  if (resident_blocks(kernel, threads) <= 0)
    return set_error(AKT_ERR_HIP, "occupancy query failed");
  int64_t blocks = wave_cap_t<D, GT>() / waves;
  const int64_t want = ceil_div(p.N > 0 ? p.N : 1, waves);
  if (blocks > want) blocks = want;
  p.W = (int)(blocks * waves);
  KernelTimer timer;
  timer.launch(kernel, dim3((unsigned)blocks), dim3(threads), 0, st, p);
  return check_launch("paged_stream_kernel");
}

template <int D>
int launch_stream_gt(int gt, const StreamParams& p, hipStream_t st) {
  switch (gt) {
    case 1: return launch_stream_t<D, 1>(p, st);
    case 2: return launch_stream_t<D, 2>(p, st);
    case 4: return launch_stream_t<D, 4>(p, st);
    case 8: return launch_stream_t<D, 8>(p, st);
    case 16:
      if constexpr (D != 256) return launch_stream_t<D, 16>(p, st);
      break;
  }
  return set_error(AKT_ERR_UNSUPPORTED, "no paged decode kernel for %d heads per unit", gt);
}

}  // namespace

bool paged_stream_eligible(int64_t batch, int64_t page_size, int64_t total_pages, int64_t Y) {
  return batch >= 1 && batch <= kStreamMaxBatch && page_size % 16 == 0 &&
         Y * total_pages * (page_size / 16) < ((int64_t)1 << 31);
}

int64_t paged_stream_wave_cap(int D, int gt) {
  switch (D) {
    case 64: return wave_cap_gt<64>(gt);
    case 128: return wave_cap_gt<128>(gt);
    case 256: return wave_cap_gt<256>(gt);
  }
  return kStreamMaxWaves;
}

int paged_stream_launch(StreamParams p, int D, int gt, hipStream_t st) {
  switch (D) {
    case 64: return launch_stream_gt<64>(gt, p, st);
    case 128: return launch_stream_gt<128>(gt, p, st);
    case 256: return launch_stream_gt<256>(gt, p, st);
  }
  return set_error(AKT_ERR_UNSUPPORTED, "head_dim %d not supported (64, 128, 256)", D);
}

}  // namespace akt
