// Selective-scan kernel parameters, lane layout and the LDS staging shared by
// the forward and backward kernels.
//
// Lane layout: a workgroup is W waves; each wave holds 4 channels (rows
// r = lane / 16) x 16 state lanes (j = lane % 16); lane j owns states
// n = j + 16 * s for s < SPL (SPL = ceil(dstate / 16)). A workgroup covers
// 4W consecutive channels of one (batch, group) slice, so all its rows share
// the same B/C rows. Time is walked in blocks of 16 steps; within a block lane
// j also "owns" step t0 + j for the per-step scalar work (softplus, gating,
// stores), and the other lanes of its row read those scalars through DPP row
// broadcasts.
//
// Staging: every per-step input of the next block (u, delta, z, dout, y and
// the B/C rows) is fetched into registers by the whole workgroup while the
// current block computes, then parked in a double-buffered LDS tile, so a
// block starts with its operands already on chip. Each tile is fetched with
// the thread index running along whichever dimension is contiguous in memory
// (time for (batch, dim, seqlen) tensors, channel for transposed views;
// state or time for B/C), which keeps the global loads coalesced for both
// the reference's layouts and Hugging Face's strided views.
#pragma once

#include "mcpu_common.h"

namespace mcpu {

constexpr int kScanBlockT = 16;       // time steps per block
constexpr int kScanRowsPerWave = 4;   // channels per wave
constexpr int kScanMaxWaves = 12;     // widest workgroup of either kernel
constexpr int kBCPad = 20;            // padded time stride of the B/C tiles (conflict-free b128 reads)
constexpr int kScanSumWaves = 4;      // waves per workgroup of the backward's chunk-summary pass

struct ScanParams {
  const void* u;
  const void* delta;
  const float* A;
  const float* B;
  const float* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  void* out;
  float* last_state;
  float* ckpt;          // (batch, dim, nblk, dstate): state at the start of each block
  void* ysave;          // (batch, dim, seqlen): y before the z gate
  const void* dout;
  const float* dlast_state;
  void* du;
  void* ddelta;
  void* dz;
  float* dA_part;       // (batch, dim, dstate)
  float* dB_part;       // (batch, ngroups, nblk_c, seqlen, dstate)
  float* dC_part;
  float* dD_part;       // (batch, dim)
  float* dbias_part;    // (batch, dim)
  int64_t batch, dim, seqlen, dstate, ngroups, dpg;
  int64_t nblk;         // ceil(seqlen / 16)
  int64_t nblk_c;       // channel blocks per slice: ceil(dpg / (4 W))
  int64_t su[3], sdl[3], sz[3], sdo[3];
  int64_t sout[3], sdu[3], sdd[3], sdz[3];  // output strides (contiguous when the caller gave none)
  int64_t sB[4], sC[4];
  int softplus;
  // Time chunks: the sequence is cut into nchunk chunks of chunk_blocks
  // 16-step blocks, scanned in parallel; chunk c starts from the state carried
  // over chunks 0..c-1 through their summaries (state at the chunk end when
  // started from zero, and the chunk's sum of dt).
  int64_t nchunk;        // 1 = unchunked
  int64_t chunk_blocks;
  float* sum_h;          // (batch, dim, nchunk, dstate); backward: (batch, dim, nsum, dstate)
  float* sum_dt;         // (batch, dim, nchunk); backward: (batch, dim, nsum)
  // Backward: adjoint summaries are kept per unit of sum_blocks blocks (nsum
  // units); a chunk is sum_per_chunk whole units.
  int64_t nsum;
  int64_t sum_blocks;
  int64_t sum_per_chunk;
  // State slices (dstate above what one lane group holds): the grid holds
  // nslices copies of the launch, copy s scanning states [s * dstate,
  // s * dstate + dstate) of the ntotal states (the last slice may be short).
  // A, ckpt, last_state, dlast_state, sum_h and the dA/dB/dC layouts keep all
  // ntotal states (nstride per row). Unsliced: nslices 1, nstride = ntotal =
  // dstate.
  int64_t nslices, nstride, ntotal;
  float* ypart;   // sliced forward: (nslices, batch, dim, seqlen) y of each slice's states
  float* rpart;   // sliced backward: (2, nslices, batch, dim, seqlen) <ga, A> and <g, B> per slice
};

// This workgroup's state slice: its index, first state and state count.
struct SliceCtx {
  int64_t sl, n0, N;
  int64_t bx;  // the workgroup's index within its slice's copy of the grid
};
__device__ __forceinline__ SliceCtx scan_slice(const ScanParams& p) {
  SliceCtx s;
  const int64_t per = gridDim.x / p.nslices;
  s.sl = blockIdx.x / per;
  s.bx = blockIdx.x % per;
  s.n0 = s.sl * p.dstate;
  s.N = p.ntotal - s.n0 < p.dstate ? p.ntotal - s.n0 : p.dstate;
  return s;
}

struct RowCtx {
  int64_t b, g, d;     // batch, group, channel (clamped into range)
  int64_t cl0;         // first channel (within the group) of the workgroup
  int64_t cblk;        // channel block of the workgroup
  bool active;         // this row's channel exists (rows past the slice end are padding)
};

// bid: the workgroup's index over (batch, group, channel block).
template <int W>
__device__ __forceinline__ RowCtx scan_row_ctx(const ScanParams& p, int64_t bid, int wave, int r) {
  RowCtx c;
  c.cblk = bid % p.nblk_c;
  bid /= p.nblk_c;
  c.g = bid % p.ngroups;
  c.b = bid / p.ngroups;
  c.cl0 = c.cblk * (4 * W);
  const int64_t cl = c.cl0 + wave * kScanRowsPerWave + r;
  c.active = cl < p.dpg;
  c.d = c.g * p.dpg + (c.active ? cl : p.dpg - 1);
  return c;
}

// One (4W channels x 16 steps) tile of a (batch, dim, seqlen) tensor. A
// thread's element is addressed as a uniform base (scalar registers), which
// moves by one block per advance(), plus a fixed per-thread 32-bit byte offset,
// so the loads use the scalar-base + vector-offset form and the running state
// costs one vector register. Channel-fastest when the channel stride is 1.
// Rows past the slice end read the slice's last channel (never out of range).
// The host guarantees (4W - 1) * |s[1]| + 15 * |s[2]| elements fit the offset.
template <int W>
struct XStage {
  const char* base;  // uniform: element (batch, first channel of the workgroup, t0)
  int32_t step;      // uniform: bytes per block (|16 * time stride| fits the 32-bit tile offsets)
  uint32_t off;      // per thread: byte offset of its element from base
  int slot;          // per thread: index c * 16 + t of its element in the LDS tile
  int t;             // per thread: its step within the block
  template <typename Tx>
  __device__ __forceinline__ void init(int tid, const void* p_base, const int64_t (&s)[3],
                                       const ScanParams& p, const RowCtx& rc, int64_t t0) {
    int c;
    if (s[1] == 1 && s[2] != 1) {
      c = tid % (4 * W);
      t = tid / (4 * W);
    } else {
      c = tid / kScanBlockT;
      t = tid % kScanBlockT;
    }
    slot = c * kScanBlockT + t;
    const int64_t last = p.dpg - 1 - rc.cl0;
    const int64_t ce = c < last ? c : last;
    constexpr int64_t sz = sizeof(Tx);
    base = static_cast<const char*>(p_base) +
           sz * (rc.b * s[0] + (rc.g * p.dpg + rc.cl0) * s[1] + t0 * s[2]);
    off = static_cast<uint32_t>(sz * (ce * s[1] + t * s[2]));
    step = static_cast<int32_t>(sz * kScanBlockT * s[2]);
  }
  // The element's bits (buf_ld_raw); raw_f32<Tx> widens them where they are
  // parked, after the block the prefetch runs under.
  template <typename Tx>
  __device__ __forceinline__ uint32_t load() const {
    return buf_ld_raw<Tx>(wave_rsrc(base), off);
  }
  // For a block that may extend past the sequence end: steps past the end
  // load the tile's first element (always in range) and read as 0. The load
  // itself is unconditional, so no prefetch register is written under a
  // lane mask (which would make the compiler drain every outstanding memory
  // operation before reusing it).
  template <typename Tx>
  __device__ __forceinline__ uint32_t load_guarded(int64_t t0, int64_t L) const {
    const bool ok = t0 + t < L;
    const uint32_t x = buf_ld_raw<Tx>(wave_rsrc(base), ok ? off : 0u);
    return ok ? x : 0u;
  }
  __device__ __forceinline__ void advance(int dir) { base += dir * step; }
  // Moves one block in direction dir unless `stay` (uniform).
  __device__ __forceinline__ void advance_unless(int dir, bool stay) { base += stay ? 0 : dir * step; }
};

// B or C rows of one block, parked transposed as [n][t] (padded) so a lane
// reads its state's 16 steps with four 16-byte LDS reads. Addressed like
// XStage: uniform base of the (batch, group) row at t0 + per-thread offset.
template <int W, int SPL>
struct BCStage {
  static constexpr int NW = 16 * SPL;
  static constexpr int PER_THREAD = (kScanBlockT * NW + 64 * W - 1) / (64 * W);
  const char* base;  // uniform
  int32_t step;      // uniform: bytes per block
  uint32_t off[PER_THREAD];
  int slot[PER_THREAD];  // n * kBCPad + t in the LDS tile, or -1 past the tile
  int t[PER_THREAD];
  bool ok[PER_THREAD];   // the state exists (n < dstate)
  // pairs: the row holds one part of (re, im) float pairs (complex B/C),
  // whose time stride is 2 in mamba_ssm's (.., dstate, 2 seqlen) layout;
  // the thread index then runs along time whenever time has the smaller
  // nonzero stride.
  __device__ __forceinline__ void init(int tid, const float* row, const int64_t (&s)[4], int64_t N,
                                       int64_t t0, bool pairs = false) {
    const bool time_fastest = pairs ? (s[2] > 0 && s[2] < s[3]) : (s[2] == 1 && s[3] != 1);
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int e = tid + i * 64 * W;
      int n;
      if (time_fastest) {  // time contiguous: time-fastest
        n = e / kScanBlockT;
        t[i] = e % kScanBlockT;
      } else {
        n = e % NW;
        t[i] = e / NW;
      }
      const bool in_tile = e < kScanBlockT * NW;
      ok[i] = in_tile && n < N;
      slot[i] = in_tile ? n * kBCPad + t[i] : -1;
      off[i] = ok[i] ? static_cast<uint32_t>(sizeof(float) * (t[i] * s[2] + n * s[3])) : 0u;
    }
    base = reinterpret_cast<const char*>(row + t0 * s[2]);
    step = static_cast<int32_t>(sizeof(float) * kScanBlockT * s[2]);
  }
  // Unconditional loads: elements outside the tile load the row's first
  // element (off = 0) and are zeroed by park(), after the block's compute, so
  // nothing consumes a prefetched value before then.
  __device__ __forceinline__ void load(float (&v)[PER_THREAD]) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) v[i] = buf_ld<float>(wave_rsrc(base), off[i]);
  }
  // Also zeroes the steps past the sequence end (see XStage::load_guarded).
  // Used for the sequence's last block only.
  __device__ __forceinline__ void load_guarded(int64_t t0, int64_t L, float (&v)[PER_THREAD]) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const bool in = ok[i] && t0 + t[i] < L;
      const float x = buf_ld<float>(wave_rsrc(base), in ? off[i] : 0u);
      v[i] = in ? x : 0.f;
    }
  }
  __device__ __forceinline__ void advance(int dir) { base += dir * step; }
  __device__ __forceinline__ void advance_unless(int dir, bool stay) { base += stay ? 0 : dir * step; }
  __device__ __forceinline__ void park(float (*tile)[kBCPad], const float (&v)[PER_THREAD]) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i)
      if (PER_THREAD * 64 * W == kScanBlockT * NW || slot[i] >= 0)
        (&tile[0][0])[slot[i]] = ok[i] ? v[i] : 0.f;
  }
};

// One partial array to sum: out[s, e] = sum over c < nsum of
// part[(s * nsum + c) * per + e], for s < outer, e < per.
struct PartialSum {
  const float* part;
  float* out;
  int64_t outer, nsum, per;
};
hipError_t partial_sums_launch(const PartialSum* sums, int n, hipStream_t stream);

// Folds chunk summaries into a state, in order: for k = 0 .. count-1 and
// c = first + dir * k, h <- exp2(A2 * sd[c]) h + sh[c * NS + n] for each of
// this lane's states n = j + 16 s < N. The summaries of a few chunks load
// together and then fold in the same order (the same arithmetic as one chunk
// at a time, without a memory round trip per chunk).
template <int SPL>
__device__ __forceinline__ void fold_summaries(float (&h)[SPL], const float (&A2)[SPL], const float* sh,
                                               const float* sd, int64_t first, int64_t count, int dir, int j,
                                               int64_t N, int64_t NS) {
  constexpr int U = SPL == 1 ? 8 : (SPL == 2 ? 4 : 2);
  for (int64_t k0 = 0; k0 < count; k0 += U) {
    float ds[U], hv[U][SPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = first + dir * (k0 + u < count ? k0 + u : count - 1);
      ds[u] = sd[c];
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const int n = j + 16 * s;
        hv[u][s] = sh[c * NS + (n < N ? n : 0)];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + u >= count) break;
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        if (j + 16 * s < N) h[s] = fmaf(fast_exp2(A2[s] * ds[u]), h[s], hv[u][s]);
    }
  }
}

// Reads the 16 steps of state lane n from a transposed B/C tile.
__device__ __forceinline__ void read_bc_row(const float (*tile)[kBCPad], int n, float (&v)[kScanBlockT]) {
  const float4* row = reinterpret_cast<const float4*>(tile[n]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 x = row[q];
    v[4 * q + 0] = x.x;
    v[4 * q + 1] = x.y;
    v[4 * q + 2] = x.z;
    v[4 * q + 3] = x.w;
  }
}

}  // namespace mcpu
