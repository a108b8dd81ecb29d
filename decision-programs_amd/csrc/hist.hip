// Node histogram construction and sibling subtraction for gfx950.
//
// The reference reaches this step only inside XGBoost's grow_gpu_hist updater
// (native/class_native_training.cuh:67).  Design for CDNA4:
//  * bins are uint8 in tiles of 16 features (tile-major: tile t holds 16 bytes
//    per row), so one lane reads the 16 bins of a row with one 128-bit load and
//    a wavefront of contiguous rows reads 1 KiB contiguous;
//  * gathered rows (levels below the root) read a row-major copy instead (all
//    tiles of a row in one run of n_tiles * 16 bytes): the workgroups of one
//    row chunk, one per tile, run together on one XCD and share every row's
//    cache lines in L2, where the tile-major layout would fetch a 64-byte
//    sector for each 16 bytes used;
//  * each workgroup privatises the histogram of one tile in 64 KiB of LDS (two
//    workgroups per CU), as int64 fixed-point sums, see hist_kernel;
//  * lane-dependent rotation of the 16 bytes keeps the 64-bit LDS atomics bank
//    conflict free for any bin values (measured: zero SQ_LDS_BANK_CONFLICT);
//  * sums are exact integers (fixed-point gradients), so the result does not
//    depend on summation order and equals the CPU restatement bit for bit;
//  * work items are row chunks x tiles, ordered so the tiles of one chunk run on
//    one XCD back to back (the chunk's gradients then come from that XCD's L2);
//  * no global atomics: a node's only chunk stores its tile straight into the
//    node histogram; chunks of larger nodes store their tile into a partial
//    slot, and hist_reduce_kernel sums the partial slots of each node and
//    derives the sibling (parent - built) in the same pass.
#include "dp_internal.hpp"
#include "gain.hpp"

#include <algorithm>
#include <mutex>

namespace dp {
namespace {

__global__ void fill_i64_kernel(int64_t* p, int64_t n, int64_t value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = value;
}

__global__ void fill_u8_kernel(uint8_t* p, int64_t n, uint8_t value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = value;
}

__global__ void iota_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = uint32_t(i);
}

// Rotates a 16-byte vector so that output byte k is input byte (k + rot) & 15.
__device__ __forceinline__ void rotate16(uint32_t w[4], uint32_t rot) {
  const uint32_t d = rot >> 2, s = rot & 3u;
  const uint32_t a0 = (d & 1u) ? w[1] : w[0];
  const uint32_t a1 = (d & 1u) ? w[2] : w[1];
  const uint32_t a2 = (d & 1u) ? w[3] : w[2];
  const uint32_t a3 = (d & 1u) ? w[0] : w[3];
  const uint32_t b0 = (d & 2u) ? a2 : a0;
  const uint32_t b1 = (d & 2u) ? a3 : a1;
  const uint32_t b2 = (d & 2u) ? a0 : a2;
  const uint32_t b3 = (d & 2u) ? a1 : a3;
  w[0] = __builtin_amdgcn_alignbyte(b1, b0, s);
  w[1] = __builtin_amdgcn_alignbyte(b2, b1, s);
  w[2] = __builtin_amdgcn_alignbyte(b3, b2, s);
  w[3] = __builtin_amdgcn_alignbyte(b0, b3, s);
}

typedef __attribute__((address_space(3))) unsigned long long lds_u64;
typedef __attribute__((address_space(3))) unsigned char lds_u8;

__device__ __forceinline__ void lds_add(lds_u64* p, unsigned long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

constexpr int kTile = 16;                // features per tile (bytes per row per tile)
constexpr int kLdsWords = 256 * 2 * kTile;  // 64 KiB of int64 per tile
constexpr int kHistThreads = 1024;

// One work item = rows [begin, end) of node `slot` for TPW consecutive
// 16-feature tiles starting at `tile` (tiles past the matrix's last are
// skipped).  LDS holds each tile's histogram as 256 rows of 256 bytes:
//   row b = [ sum qg of features 0..15 | sum qh of features 0..15 ] (int64 each)
// so the word of (b, f) is at byte b*256 + f*8 (g) and +128 (h); tile j of
// the item at j * 64 KiB.  A lane owns one matrix row per pipeline step: one
// 128-bit load per tile brings its 16 bin bytes.  The bytes are rotated by
// (lane & 15) so that at every one of the 16 steps the 16 lanes of a group
// address 16 distinct features, i.e. 16 distinct bank pairs (f*8 mod 128),
// whatever their bins: the 64-bit LDS atomics are conflict free.  The LDS
// address is assembled by one v_perm_b32: byte 1 = the bin byte, byte 0 = the
// lane's feature offset for that step.
//
// TPW (tiles per work item, 1 or 2) and U (rows per lane per pipeline step, 1
// or 2) are the autotuner's choices: two tiles per item read each row's
// gradient pair once for 32 features (half the re-reads of TPW 1) with 128
// KiB of LDS and one workgroup per CU; one tile per item fits two workgroups
// per CU.
//
// The row loads have no branches, so the compiler's memory counters see a
// straight pipeline: indices past `end` are clamped to the last row and their
// (g, h) masked to zero.  With MISSING, lanes whose byte is 255 (missing; such
// matrices have at most 255 bins) skip the atomics by exec mask, which keeps
// sparse data (C5: 95 % missing) from spending LDS cycles on absent values.
// The rows of an item are taken in blocks of kHistThreads * U, through a ring
// of PD + 1 register buffers: while a block is accumulated, the bins and
// gradients of the next PD blocks are in flight (PD: the prefetch depth), and
// gathered rows (GATHER) load their row ids PD + 1 blocks ahead of their data.
// Loads return in order for the memory counter, so waiting for a row id also
// waits for every older load; the row id of block j is issued after the data
// of block j - PD - 1, which is accumulated before block j's data is issued,
// so that wait costs nothing.  DEEP false: PD 1 for gathered rows, 0 for
// contiguous rows (loaded and accumulated block by block; with two resident
// workgroups per CU the other workgroup's waves hide the load latency).  DEEP
// true: PD 3, which keeps about 3 * 1024 rows of loads in flight per workgroup
// -- what the measured load latency of the gathered levels needs at the LDS
// rate when a level has fewer items than CUs (one workgroup per CU, nothing
// else to hide the latency).  DEEP costs registers (two workgroups per CU may
// no longer fit; the launcher reads the occupancy).  Blocks past the item's
// end are loaded clamped (in bounds) and not accumulated.  Workgroups loop
// over items (item = blockIdx.x + k * gridDim.x); with a grid that is a
// multiple of 8, item i still runs on XCD i mod 8.
//
// SPLIT (two tiles per item only; 0, 4 or 5): lanes whose bit SPLIT of the
// lane index is set take the item's two tiles in the other order.  Each
// 64-bit atomic instruction then updates 32 features, each from two lanes
// instead of four, which halves the lanes that can collide on one (feature,
// bin) -- the same-address conflicts of features with few live bins.  Bit 4
// alternates 16-lane rows, bit 5 splits the wavefront into halves.
//
// MODE 2 (matrices without missing values): `skip` holds, per tile, the 16
// features' most frequent bins; a lane whose byte equals its feature's skip
// bin issues no atomics (the bin's sums are the node's totals minus the other
// bins', which the split evaluation restores).  On data dominated by one value
// per feature (C4's zero pixels) this removes most atomics and their
// same-address conflicts.  MODE 1 is the missing-byte skip above; MODE 0 none.
// PAIR (items without missing values or skip bins; one tile per item, or two
// whose tiles are the pair): the item covers
// tiles t and t + 1 of dp_bin_layout::paired_tiles, whose bins are all below
// 16, and reads their joint tile (per row and feature slot i the byte tile
// t's bin << 4 | tile t + 1's bin: stored after the matrix's tiles, and in
// place of tile t in the row-major copy of gathered passes), so the
// row's 32 features cost one 16-byte load and the 16 atomic pairs of one tile:
// an ordinary item's work.  The flush takes the marginals: tile t's bin a is
// the sum of joint bins 16 a .. 16 a + 15, tile t + 1's bin b the sum of joint
// bins b, b + 16, ... (one word per thread, 16 LDS reads), and bins 16 and up
// of both tiles are zero.  Both tiles' outputs have the layout of two ordinary
// items.
struct HistPass {
  const uint8_t* bins;
  const uint8_t* skip;
  int32_t n_features, n_tiles;
  const int2* gpair;
  const uint32_t* ridx;
  int32_t bin_stride;
  unsigned long long* hist;
  unsigned long long* partial;
  int64_t tile_step, row_step;
  int32_t fmaj;
};

// src_tile: the tile whose bytes the item reads (w.tile, or a pair's joint tile).
template <bool GATHER, int MODE, int TPW, int U, int SPLIT, bool DEEP, bool PAIR>
__device__ __forceinline__ void hist_item(const HistPass& a, const HistWork& w, int32_t src_tile,
                                          unsigned long long* lds, const uint32_t (&slotw)[4],
                                          uint32_t rot) {
  static_assert(!PAIR || MODE == 0, "pairs take items without skips");
  constexpr int64_t kStep = int64_t(kHistThreads) * U;
  constexpr int PD = DEEP ? 3 : (GATHER ? 1 : 0);  // prefetch depth (blocks)
  constexpr int R = PD + 1;                         // ring buffers
  constexpr int TW = PAIR ? 1 : TPW;                // tiles read per row (a pair: its joint tile)
  lds_u8* const lds_base = (lds_u8*)lds;
  // tiles of this item that exist (uniform per workgroup); a pair fills one LDS tile
  const int nt = TW == 1 ? 1 : (w.tile + TPW <= a.n_tiles ? TPW : a.n_tiles - w.tile);
  // This lane's tile order: swapped when SPLIT applies and both tiles exist.
  const int swap = (SPLIT > 0 && nt == 2) ? int((threadIdx.x >> SPLIT) & 1u) : 0;
  // MODE 2: each tile's skip bins, rotated like the row bytes (byte k of the
  // rotated vector is the skip bin of the feature this lane takes at step k).
  uint32_t sk[TPW][4];
  if constexpr (MODE == 2) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const uint4 s4 = *reinterpret_cast<const uint4*>(
          a.skip + int64_t(w.tile + (j < nt ? j ^ swap : 0)) * kTile);
      sk[j][0] = s4.x;
      sk[j][1] = s4.y;
      sk[j][2] = s4.z;
      sk[j][3] = s4.w;
      rotate16(sk[j], rot);
    }
  }
  const uint8_t* tile = a.bins + int64_t(src_tile) * a.tile_step;  // row r at tile + r * row_step
  const int64_t last = w.end - 1;
  const int64_t lane = threadIdx.x;
  uint32_t rows[R][U];  // GATHER: row ids
  uint4 v[R][U][TW];
  int2 q[R][U];
  auto fetch_rows = [&](int b, int64_t base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + int64_t(u) * kHistThreads + lane;
      rows[b][u] = a.ridx[i < w.end ? i : last];
    }
  };
  auto fetch_data = [&](int b, int64_t base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + int64_t(u) * kHistThreads + lane;
      const uint32_t r = GATHER ? rows[b][u] : uint32_t(i < w.end ? i : last);
      const uint8_t* src = tile + int64_t(r) * a.row_step;
#pragma unroll
      for (int j = 0; j < TW; ++j)  // a missing second tile re-reads the first
        v[b][u][j] = *reinterpret_cast<const uint4*>(src + (j < nt ? j ^ swap : 0) * a.tile_step);
      q[b][u] = a.gpair[r];
    }
  };
  auto process = [&](int b, int64_t base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = base + int64_t(u) * kHistThreads + lane < w.end;
      const unsigned long long g = ok ? (unsigned long long)(long long)q[b][u].x : 0ull;
      const unsigned long long h = ok ? (unsigned long long)(long long)q[b][u].y : 0ull;
#pragma unroll
      for (int j = 0; j < TW; ++j) {
        if (j >= nt) break;  // uniform per workgroup
        uint32_t x[4] = {v[b][u][j].x, v[b][u][j].y, v[b][u][j].z, v[b][u][j].w};
        rotate16(x, rot);
        lds_u8* const base_j = lds_base + (j ^ swap) * (kLdsWords * 8);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const uint32_t sel = 0x0c0c0000u | ((4u + uint32_t(k & 3)) << 8) | uint32_t(k & 3);
          const uint32_t off = __builtin_amdgcn_perm(x[k >> 2], slotw[k >> 2], sel);
          if (MODE == 1 && off >= 255u * 256u) continue;  // byte 255: missing value
          if (MODE == 2 && off == __builtin_amdgcn_perm(sk[j][k >> 2], slotw[k >> 2], sel))
            continue;  // the feature's skip bin
          lds_u64* p = (lds_u64*)(base_j + off);
          lds_add(p, g);
          lds_add(p + 16, h);
        }
      }
    }
  };
  // The loop bound and the block guards are uniform per workgroup; buffer
  // indices are static (buffer j % R holds block j of the item).  The item's
  // first loads are issued before the LDS clear and its barrier, which they
  // do not depend on (a barrier waits for LDS operations only), so the clear
  // runs while they are in flight.
  const int64_t b0 = w.begin;
  if (GATHER) {
#pragma unroll
    for (int j = 0; j < R; ++j) fetch_rows(j, b0 + j * kStep);
  }
  for (int e = threadIdx.x; e < nt * kLdsWords; e += kHistThreads) lds[e] = 0ull;
  if (GATHER) {
#pragma unroll
    for (int j = 0; j < PD; ++j) {
      fetch_data(j, b0 + j * kStep);
      fetch_rows(j, b0 + (j + R) * kStep);
    }
  } else {
#pragma unroll
    for (int j = 0; j < PD; ++j) fetch_data(j, b0 + j * kStep);
  }
  __syncthreads();
  for (int64_t blk = b0; blk < w.end; blk += R * kStep) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int n = (k + PD) % R;  // the buffer of block k + PD
      fetch_data(n, blk + (k + PD) * kStep);
      if (GATHER) fetch_rows(n, blk + (k + PD + R) * kStep);
      if (k == 0 || blk + k * kStep < w.end) process(k, blk + k * kStep);
    }
  }
  __syncthreads();

  const int n_words = a.bin_stride * 32;  // bins < bin_stride, 32 words each
  if constexpr (PAIR) {
    static_assert(kHistThreads == 1024, "one marginal word per thread");
    // Thread e: output tile jj = e / 512 (0: tile t, 1: tile t + 1), bin x,
    // word c of the LDS row layout (g of the 16 features, then h).  e is
    // opaque to the compiler here, so that nothing derived from it is hoisted
    // out of the item loop and held in registers across the row loop.
    int e = int(threadIdx.x);
    __asm__ volatile("" : "+v"(e));
    const int jj = e >> 9, x = (e >> 5) & 15, c = e & 31;
    unsigned long long m = 0;
#pragma unroll 2
    for (int y = 0; y < 16; ++y) m += lds[(jj ? 16 * y + x : 16 * x + y) * 32 + c];
    // Tile jj's output: the partial slot w.partial + jj (LDS image or
    // feature-major) or, for a direct item, its features of node w.slot.
    const bool image = w.partial >= 0 && !a.fmaj;
    const int64_t node_words = int64_t(a.n_features) * a.bin_stride * 2;
    // off: the word within the image, else within feature fi's bins.
    auto put = [&](int t, int fi, int off, unsigned long long val) {
      if (image) {
        a.partial[int64_t(w.partial + t) * n_words + off] = val;
      } else if (w.partial >= 0) {
        a.partial[int64_t(w.partial + t) * n_words + int64_t(fi) * a.bin_stride * 2 + off] = val;
      } else {
        const int f = (w.tile + t) * kTile + fi;
        if (f < a.n_features)
          a.hist[int64_t(w.slot) * node_words + int64_t(f) * a.bin_stride * 2 + off] = val;
      }
    };
    if (x < a.bin_stride) put(jj, c & 15, image ? x * 32 + c : x * 2 + (c >> 4), m);
    // bins 16 .. bin_stride - 1 of both tiles: zero
    const int zb = a.bin_stride > 16 ? a.bin_stride - 16 : 0;
    if (image) {  // rows 16 and up: one run of zb * 32 words per tile
      for (int z = e; z < 2 * zb * 32; z += kHistThreads) {
        const int t = z >= zb * 32 ? 1 : 0;
        put(t, 0, 16 * 32 + (z - t * zb * 32), 0ull);
      }
    } else {  // per feature: a run of zb * 2 words from bin 16
      const int per = zb * 2;
      for (int z = e; z < 2 * 16 * per; z += kHistThreads) {
        const int t = z >= 16 * per ? 1 : 0, r = z - t * 16 * per, fi = r / per;
        put(t, fi, 32 + (r - fi * per), 0ull);
      }
    }
  } else {
    for (int j = 0; j < nt; ++j) {
      const unsigned long long* src = lds + j * kLdsWords;
      if (w.partial >= 0 && a.fmaj) {  // feature-major partial slot: [16][bin_stride][g, h]
        // Pair q = (bin q / 16, feature q % 16): its (g, h) words, 16 bytes at
        // (feature * bin_stride + bin) * 2.  One store instruction of a
        // wavefront writes four bins of 16 features, a 64-byte run per feature;
        // the LDS reads of one feature's four bins share a bank pair (4-way).
        auto* out = reinterpret_cast<ulonglong2*>(a.partial + int64_t(w.partial + j) * n_words);
        for (int q = threadIdx.x; q < 16 * a.bin_stride; q += kHistThreads) {
          const int fl = q & 15, b = q >> 4;
          out[fl * a.bin_stride + b] = make_ulonglong2(src[b * 32 + fl], src[b * 32 + 16 + fl]);
        }
      } else if (w.partial >= 0) {  // tile j's partial slot is the item's slot + j (LDS image)
        unsigned long long* out = a.partial + int64_t(w.partial + j) * n_words;
        for (int e = threadIdx.x; e < n_words; e += kHistThreads) out[e] = src[e];
      } else {
        unsigned long long* out = a.hist + int64_t(w.slot) * a.n_features * a.bin_stride * 2;
        const int f0 = (w.tile + j) * kTile;
        for (int e = threadIdx.x; e < n_words; e += kHistThreads) {
          const int bin = e >> 5, within = e & 31;
          const int f = f0 + (within & 15);
          if (f < a.n_features)
            out[(int64_t(f) * a.bin_stride + bin) * 2 + (within >> 4)] = src[e];
        }
      }
    }
  }
  __syncthreads();  // the next item clears the LDS this item just read
}

// PAIRS: the launch has paired tiles (an instantiation of its own, so that the
// kernels of unpaired launches carry no pair items' code or registers).
template <bool GATHER, int MODE, int TPW, int U, int SPLIT = 0, bool DEEP = false,
          bool PAIRS = false>
__global__ __launch_bounds__(kHistThreads) __attribute__((amdgpu_waves_per_eu(DEEP && !(PAIRS && U == 1) ? 4 : 8 / TPW, 8 / TPW))) void hist_kernel(
    const uint8_t* __restrict__ bins, const uint8_t* __restrict__ skip, int64_t n_rows,
    int32_t n_features, int32_t n_tiles,
    const int2* __restrict__ gpair, const uint32_t* __restrict__ ridx,
    const HistWork* __restrict__ work, int32_t n_work_host,
    const int32_t* __restrict__ n_work_dev, int32_t bin_stride,
    unsigned long long* __restrict__ hist, unsigned long long* __restrict__ partial,
    int64_t tile_step, int64_t row_step, int32_t fmaj, uint64_t pairs, uint64_t joint_pairs,
    int32_t joint_first) {
  extern __shared__ unsigned long long lds[];  // TPW * kLdsWords
  // The first item is loaded alongside the device count (the host bound keeps
  // it in range), so the two loads overlap instead of chaining.
  const HistWork w_first =
      int32_t(blockIdx.x) < n_work_host ? work[blockIdx.x] : HistWork{0, 0, 0, 0, -1, 0};
  const int32_t n_work = n_work_dev ? *n_work_dev : n_work_host;
  const uint32_t rot = threadIdx.x & 15u;
  uint32_t slotw[4];  // byte i of slotw[m]: feature offset (bytes) of step 4m+i
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) v |= (((uint32_t(4 * m + i) + rot) & 15u) * 8u) << (8 * i);
    slotw[m] = v;
  }
  (void)n_rows;
  const HistPass a{bins, skip, n_features, n_tiles, gpair, ridx, bin_stride, hist, partial,
                   tile_step, row_step, fmaj};
  for (int32_t item = blockIdx.x; item < n_work; item += gridDim.x) {
    const HistWork w = item == int32_t(blockIdx.x) ? w_first : work[item];
    if (w.begin >= w.end) continue;  // padding item (uniform per workgroup)
    if constexpr (PAIRS) {
      static_assert(MODE == 0, "pairs take items without skips");
      if (w.tile < 63 && ((pairs >> w.tile) & 1ull)) {  // the item's tiles are pair k
        const int32_t k = __builtin_popcountll(joint_pairs & ((1ull << w.tile) - 1ull));
        const int32_t jt = joint_first < 0 ? w.tile : joint_first + k;  // its joint tile
        hist_item<GATHER, MODE, TPW, U, SPLIT, DEEP, true>(a, w, jt, lds, slotw, rot);
        continue;
      }
    }
    hist_item<GATHER, MODE, TPW, U, SPLIT, DEEP, false>(a, w, w.tile, lds, slotw, rot);
  }
}

// The evaluation a present-value pass does for its single-chunk nodes (EVAL).
struct SparseEvalArgs {
  const long long* parent_base;  // previous level's node histograms
  const int32_t* n_bins;
  const long long* node_sums;
  const int32_t* exps;
  Param p;
  const uint32_t* fmask;
  const uint8_t* skip_bins;
  FeatCand* cand;
  int32_t store;  // 0: the level's histograms have no readers (nothing stored)
};

// EVAL's epilogue (see hist_sparse_kernel): node w.slot's features f0 .. f0 +
// nf from the LDS planes (g, h: [feature][bin_stride + 1] words), and its sibling's from
// the parent's words minus them; every thread of the workgroup takes part.
// The lane's bins are evaluated one after the other (seg_evaluate<true>):
// interleaving their divisions needs more than the 128 registers of two such
// workgroups per CU.
template <int THREADS>
__device__ __forceinline__ void evaluate_tile(const SparseEvalArgs& ev, const HistWork& w,
                                              int32_t f0, int32_t nf, int32_t n_features,
                                              int32_t bin_stride, const unsigned long long* lds,
                                              uint32_t ps, uint32_t hoff,
                                              unsigned long long* __restrict__ hist,
                                              long long* __restrict__ scr) {
  constexpr int BPL = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seg = lane >> 4, sub = lane & 15;
  const double ug = ldexp(1.0, -ev.exps[0]), uh = ldexp(1.0, -ev.exps[1]);
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  const bool sib = w.parent >= 0;  // uniform per workgroup
  // This lane's four bins of feature fl from the LDS planes (zero past the bins).
  auto load = [&](int32_t fl, bool live, long long (&g)[BPL], long long (&h)[BPL]) {
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int b = sub * BPL + k;
      const bool ok = live && b < bin_stride;
      const uint32_t a = uint32_t(live ? fl : 0) * ps + uint32_t(ok ? b : 0);
      g[k] = ok ? (long long)lds[a] : 0;
      h[k] = ok ? (long long)lds[a + hoff] : 0;
    }
  };
  for (int32_t fb = 0; fb < nf; fb += (THREADS / 64) * 4) {
    const int32_t fl = fb + wave * 4 + seg;
    const bool live = fl < nf;
    const int64_t at = (int64_t(f0 + (live ? fl : 0)) * bin_stride + sub * BPL) * 2;
    // The parent's words are loaded first, so that their latency is hidden by
    // the node's evaluation.
    long long pg[BPL], ph[BPL];
    if (sib) {
      const long long* par = ev.parent_base + int64_t(w.parent) * node_elems + at;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const bool ok = live && sub * BPL + k < bin_stride;
        pg[k] = ok ? par[2 * k] : 0;
        ph[k] = ok ? par[2 * k + 1] : 0;
      }
    }
    long long g[BPL], h[BPL];
    load(fl, live, g, h);
    seg_evaluate<true>(g, h, w.slot, f0 + fl, live, n_features, ev.n_bins, ev.node_sums, ug, uh,
                       ev.p, ev.fmask, ev.skip_bins, ev.cand, scr);
    if (!sib) continue;
    // The sibling: the parent's words minus the node's (read again from LDS,
    // so that they are not held across the evaluation above).
    load(fl, live, g, h);
    long long* so = reinterpret_cast<long long*>(hist) + int64_t(w.slot ^ 1) * node_elems + at;
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const bool ok = live && sub * BPL + k < bin_stride;
      g[k] = ok ? pg[k] - g[k] : 0;
      h[k] = ok ? ph[k] - h[k] : 0;
      if (ok && ev.store) {
        so[2 * k] = g[k];
        so[2 * k + 1] = h[k];
      }
    }
    seg_evaluate<true>(g, h, w.slot ^ 1, f0 + fl, live, n_features, ev.n_bins, ev.node_sums, ug,
                       uh, ev.p, ev.fmask, ev.skip_bins, ev.cand, scr);
  }
}

// Histograms from the present-value layout (SparseBins): one work item = rows
// [begin, end) of node `slot` for one sparse tile of tile_features features.
// Contiguous rows (the root) read the tile-major entries; gathered rows read
// the row-major copy, whose (row, tile) ranges of one row are adjacent, so the
// tile items of a row chunk, dispatched on one XCD, share each row's offsets
// and entries in L2.
// The tile's histogram lives in LDS as two planes, g then h, each
// [feature][bin_stride + 1] int64 (dynamic LDS; the h plane at the fixed word
// kSparsePlaneWords): a plane's words of one feature are adjacent, so the
// 64-bit atomics of a wavefront spread over the banks by bin, and the one-word
// pad per feature shifts each feature's bins by one bank pair, so that
// features spread them too.  An entry is its word's index in a plane, so its
// two atomics need one address.  The store interleaves the planes into the
// node histogram's [feature][bin][g, h] layout.
//
// The entries are spread over the lanes, not the rows: a wavefront takes 64
// rows at a time (rows begin + 64 (k * waves + wave) + lane), loads their
// entry ranges and (g, h), and scans the ranges' lengths (a DPP scan) into
// each row's first position in the rows' concatenated entries.  It then
// takes those entries 128 positions per round, two adjacent ones per lane:
// the rows whose first position falls in the round's window write their lane
// into the wavefront's map (one word per position, tagged with the round so
// that stale words from earlier rounds are ignored and nothing needs
// clearing), every lane reads its two positions' words, and a DPP max-scan
// carries each row to the positions after its first (rows increase with
// position).  The lane then takes (g, h), and for gathered rows the entry
// range's start, from the row's lane (ds_bpermute) and adds its entries.
// Every lane thus does the same work whatever the rows' lengths (a per-row
// walk runs at the pace of the wavefront's fullest row: 3.2 present values
// per 64-feature tile on average at C5's density, up to 12), and on the root
// pass the rows' entries are one contiguous run, read with coalesced loads.
// LDS operations of one wavefront execute in order, so a lane reads the map
// words other lanes wrote just before.  Per-lane trip counts are uniform; no
// barrier sits inside the row loop.
//
// EVAL: an item that is its node's only chunk (partial < 0) also evaluates
// the node from the LDS tile, and its sibling (parent >= 0; the sibling is
// slot ^ 1) as the parent's tile minus it --
// the words and per-feature candidates of reduce_evaluate_flat_kernel, which
// then skips the node's job.  Sixteen wavefronts take 64 of the tile's
// features per step, one per 16-lane row with four bins per lane
// (seg_evaluate).  The node's words (and the sibling's) are stored only with
// ev.store, so on the tree's last split level such a node never leaves LDS.
// Entry positions per lane and round: four on contiguous rows (one aligned
// 8-byte load), two on gathered rows (each position its own load and row base).
template <bool GATHER>
constexpr int kPosPerLane = GATHER ? 2 : 4;
constexpr int kMapSlotsMax = 64 * 4;  // positions per round and wavefront, at most
// Map word (16 bits): round tag << 8 | lane.  Tags run 0 .. kMapTagWrap - 1;
// 0xffff marks a word no round has written.
constexpr uint32_t kMapTagWrap = 255;
// EVAL's workgroups: 512 threads, so that the evaluation's double arithmetic
// has 128 registers without spilling while two workgroups share a CU.
constexpr int kSparseEvalThreads = 512;

// Inclusive max over the wavefront's lanes of non-negative values (row_shr 1,
// 2, 4, 8, then row_bcast15 and row_bcast31; a lane without a source takes 0,
// the identity, so each step is one max with a DPP operand).
__device__ __forceinline__ uint32_t wave_inclusive_umax(uint32_t x) {
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x111, 0xf, 0xf, false)));
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x112, 0xf, 0xf, false)));
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x114, 0xf, 0xf, false)));
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x118, 0xf, 0xf, false)));
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x142, 0xa, 0xf, false)));
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x143, 0xc, 0xf, false)));
  return x;
}

template <bool GATHER, bool EVAL, int THREADS>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(4))) void
hist_sparse_kernel(
    const uint32_t* __restrict__ ptr, const uint16_t* __restrict__ entries, int64_t n_rows,
    int32_t n_features, int32_t tile_features, const int2* __restrict__ gpair,
    const uint32_t* __restrict__ ridx, const HistWork* __restrict__ work, int32_t n_work_host,
    const int32_t* __restrict__ n_work_dev, int32_t bin_stride,
    unsigned long long* __restrict__ hist, unsigned long long* __restrict__ partial,
    SparseEvalArgs ev, int32_t ptr_rows) {
  extern __shared__ unsigned long long lds_tile[];  // g plane, then h plane
  constexpr int P = kPosPerLane<GATHER>;
  constexpr int kMapSlots = 64 * P;  // positions per round
  // Each wavefront's map of one round's kMapSlots positions (16-bit words,
  // 8-byte aligned for the lanes' wide reads).  With EVAL the same words are
  // also the wavefront's scratch of seg_evaluate (cleared after it).
  constexpr int kMapWords = EVAL ? kSegScratchWords : kMapSlotsMax / 4;
  static_assert(kMapWords >= kMapSlotsMax / 4, "the map fits its wavefront's words");
  __shared__ __attribute__((aligned(16))) uint2 lds_map[THREADS / 64][kMapWords];
  const int32_t n_work = n_work_dev ? *n_work_dev : n_work_host;
  const int64_t slot_words = int64_t(tile_features) * bin_stride * 2;
  const uint32_t ps = uint32_t(bin_stride) + 1u;         // plane words per feature
  constexpr uint32_t hoff = uint32_t(kSparsePlaneStride);  // the h plane's offset
  const unsigned long long* const lds_h = lds_tile + hoff;
  const uint32_t plane = uint32_t(tile_features) * ps;   // live words of a plane
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // lane l's words: positions P l .. P l + P - 1
  uint16_t* const map = reinterpret_cast<uint16_t*>(lds_map[wave]);
  // This lane's P words, read and cleared as one 4- or 8-byte access.
  auto read_words = [&](uint32_t (&word)[4]) {
    if constexpr (P == 4) {
      const uint2 m = reinterpret_cast<const uint2*>(map)[lane];
      word[0] = m.x & 0xffffu;
      word[1] = m.x >> 16;
      word[2] = m.y & 0xffffu;
      word[3] = m.y >> 16;
    } else {
      const uint32_t m = reinterpret_cast<const uint32_t*>(map)[lane];
      word[0] = m & 0xffffu;
      word[1] = m >> 16;
    }
  };
  auto clear_words = [&] {
    if constexpr (P == 4) reinterpret_cast<uint2*>(map)[lane] = make_uint2(~0u, ~0u);
    else reinterpret_cast<uint32_t*>(map)[lane] = ~0u;
  };
  clear_words();  // no round has written a word yet
  uint32_t tag = 0;
  // A masked position adds its values to the trash word of its lane.
  const uint32_t trash = uint32_t(kSparsePlaneWords) + uint32_t(lane);
  for (int32_t item = blockIdx.x; item < n_work; item += gridDim.x) {
    const HistWork w = work[item];
    if (w.begin >= w.end) continue;  // padding item (uniform per workgroup)
    const int32_t f0 = w.tile * tile_features;
    const int32_t nf = f0 + tile_features < n_features ? tile_features : n_features - f0;
    for (uint32_t e = threadIdx.x; e < plane; e += THREADS) {
      lds_tile[e] = 0ull;
      lds_tile[hoff + e] = 0ull;
    }
    __syncthreads();
    // (tile t, row r)'s entry range starts at ptr[t * n_rows + r] in the
    // tile-major layout (ptr_rows 1), at ptr[r * ptr_rows + t] in the row-major
    // copy (ptr_rows = n_tiles; gathered rows only).
    const int64_t rstep = GATHER ? ptr_rows : 1;
    const uint32_t* tp = ptr + int64_t(w.tile) * (rstep == 1 ? n_rows : 1);
    // The rows of block i0 (rows i0 + lane): entry range start, length and
    // (g, h), loaded one block ahead (gathered row ids two blocks ahead).
    // Loads are branch-free (indexes past the item clamped, their values
    // masked), so that the compiler counts them and waits only for the ones a
    // step needs.
    struct Rows {
      uint32_t b, c;
      int2 q;
    };
    auto row_id = [&](int64_t i0) -> uint32_t {
      const int64_t i = i0 + lane;
      return GATHER ? ridx[i < w.end ? i : w.end - 1] : uint32_t(i < w.end ? i : w.end - 1);
    };
    auto load_rows = [&](int64_t i0, uint32_t r) -> Rows {
      const bool valid = i0 + lane < w.end;
      const uint32_t b = tp[int64_t(r) * rstep], e = tp[int64_t(r) * rstep + 1];
      const int2 q = gpair[r];
      return Rows{b, valid ? e - b : 0u, valid ? q : make_int2(0, 0)};
    };
    int64_t i0 = w.begin + int64_t(wave) * 64;
    uint32_t r_ahead = GATHER ? row_id(i0 + THREADS) : 0u;
    Rows cur = load_rows(i0, row_id(i0));
    for (; i0 < w.end; i0 += THREADS) {
      const Rows nxt = load_rows(i0 + THREADS, GATHER ? r_ahead : row_id(i0 + THREADS));
      if (GATHER) r_ahead = row_id(i0 + 2 * THREADS);
      const int c = int(cur.c);
      const int incl = wave_inclusive_sum32(c);
      uint32_t first = uint32_t(incl - c);  // the row's first position
      uint32_t total = uint32_t(__builtin_amdgcn_readlane(incl, 63));
      // Gathered rows: position p of row v is entry base_v + p.
      const uint32_t base = cur.b - first;
      // Contiguous rows: the block's entries are one run from lane 0's b.
      // Positions count from that entry rounded down to a multiple of 4
      // (`shift` positions of the block before, masked), so that a lane's
      // four positions are one aligned 8-byte load.
      uint32_t shift = 0, a0 = 0;
      if (!GATHER) {
        const uint32_t b0 = uint32_t(__builtin_amdgcn_readfirstlane(cur.b));
        shift = b0 & 3u;
        a0 = b0 - shift;
        first += shift;
        total = total ? total + shift : 0u;
      }
      uint32_t carry = 0;  // the row of the position before the round's window
      for (uint32_t j = 0; j < total; j += kMapSlots) {
        // Rows whose first position falls in [j, j + kMapSlots) mark it.
        if (c > 0 && first - j < uint32_t(kMapSlots)) map[first - j] = uint16_t(tag << 8 | lane);
        __builtin_amdgcn_wave_barrier();
        uint32_t word[4];
        read_words(word);
        __builtin_amdgcn_wave_barrier();
        uint32_t run = 0, row[P];
#pragma unroll
        for (int k = 0; k < P; ++k) {
          run = max(run, (word[k] >> 8) == tag ? (word[k] & 63u) : 0u);
          row[k] = run;
        }
        const uint32_t scan = wave_inclusive_umax(max(run, carry));
        // the lanes before's rows (lane 0: the carry) bound this lane's
        const uint32_t before =
            uint32_t(__builtin_amdgcn_update_dpp(int(carry), int(scan), 0x138, 0xf, 0xf, false));
        carry = uint32_t(__builtin_amdgcn_readlane(int(scan), 63));
        if (++tag == kMapTagWrap) {  // uniform: start the tags again on a clean map
          clear_words();
          tag = 0;
        }
        const uint32_t p = j + uint32_t(P * lane);  // this lane's first position
        uint32_t x[P];
        if constexpr (!GATHER) {  // one aligned load of the four entries (past the end: a0's)
          const uint2 v = *reinterpret_cast<const uint2*>(entries + a0 + (p < total ? p : 0u));
          x[0] = v.x & 0xffffu;
          x[1] = v.x >> 16;
          x[2] = v.y & 0xffffu;
          x[3] = v.y >> 16;
        }
#pragma unroll
        for (int k = 0; k < P; ++k) {
          const int vk = int(max(row[k], before));
          const uint32_t pk = p + uint32_t(k);
          const bool in = pk < total && pk >= shift;
          // Every lane takes part in the row lane reads (a lane reads the value
          // of another lane only while both are active), so they come before
          // any masking.
          const int g = __shfl(cur.q.x, vk, 64), h = __shfl(cur.q.y, vk, 64);
          if (GATHER) {
            const uint32_t bv = uint32_t(__shfl(int(base), vk, 64));
            x[k] = entries[in ? bv + pk : 0u];
          }
          lds_u64* const at = (lds_u64*)lds_tile + (in ? x[k] : trash);
          lds_add(at, (unsigned long long)(long long)g);
          lds_add(at + hoff, (unsigned long long)(long long)h);
        }
      }
      cur = nxt;
    }
    __syncthreads();
    const bool direct = w.partial < 0;  // uniform per workgroup
    unsigned long long* out =
        !direct ? partial + int64_t(w.partial) * slot_words
                : hist + (int64_t(w.slot) * n_features + f0) * bin_stride * 2;
    if (!(EVAL && direct && !ev.store))
      for (int k = threadIdx.x; k < nf * bin_stride; k += THREADS) {  // (feature, bin) pairs
        const int32_t f = k / bin_stride, a = f * int32_t(ps) + (k - f * bin_stride);
        reinterpret_cast<ulonglong2*>(out)[k] = make_ulonglong2(lds_tile[a], lds_h[a]);
      }
    if constexpr (EVAL) {
      if (direct) {
        evaluate_tile<THREADS>(ev, w, f0, nf, n_features, bin_stride, lds_tile, ps, hoff, hist,
                               reinterpret_cast<long long*>(lds_map[wave]));
        // The scratch overwrote the map words: none may carry a live tag.
        __builtin_amdgcn_wave_barrier();
        clear_words();
      }
    }
    __syncthreads();  // the next item clears the LDS this item just read
  }
}

// Sum of nc partial-slot words src[k * step], k < nc, exact in int64: eight
// loads in flight per thread (unguarded blocks of eight, then four, then one;
// measured: per-load guards inside one unrolled loop serialise the loads).
__device__ __forceinline__ long long sum_slots(const long long* __restrict__ src, int64_t step,
                                               int32_t nc) {
  long long acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int32_t k = 0;
  for (; k + 8 <= nc; k += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += src[(k + u) * step];
  }
  if (k + 4 <= nc) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += src[(k + u) * step];
    k += 4;
  }
  for (; k < nc; ++k) acc[4] += src[k * step];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// Reduce for the present-value path: partial slots hold a sparse tile in the
// node histogram's layout, so word e of tile t is word t * tile_features *
// bin_stride * 2 + e of the node histogram.  Otherwise as hist_reduce_kernel.
__global__ __launch_bounds__(256) void hist_reduce_flat_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs,
    int32_t n_jobs_host, const int32_t* __restrict__ n_jobs_dev, int32_t n_tiles,
    int32_t tile_features, int32_t n_features, int32_t bin_stride,
    const long long* __restrict__ parent_base, long long* __restrict__ hist) {
  const int32_t n_jobs = n_jobs_dev ? *n_jobs_dev : n_jobs_host;
  const int t = blockIdx.y;
  const int32_t f0 = t * tile_features;
  const int32_t nf = f0 + tile_features < n_features ? tile_features : n_features - f0;
  const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (e >= int64_t(nf) * bin_stride * 2) return;  // no barriers below
  const int64_t slot_words = int64_t(tile_features) * bin_stride * 2;
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  const int64_t at = int64_t(f0) * bin_stride * 2 + e;
  for (int32_t jb = blockIdx.z; jb < n_jobs; jb += gridDim.z) {
    const HistReduce j = jobs[jb];
    long long* built = hist + int64_t(j.slot) * node_elems + at;
    long long sum;
    if (j.nc == 1 && j.p0 < 0) {
      sum = *built;  // written directly by the node's only chunk
    } else {
      sum = sum_slots(partial + (int64_t(j.p0) * n_tiles + t) * slot_words + e,
                      int64_t(n_tiles) * slot_words, j.nc);
      *built = sum;
    }
    if (j.sibling >= 0)
      hist[int64_t(j.sibling) * node_elems + at] = parent_base[j.parent + at] - sum;
  }
}

__global__ void zero_i64_dev_kernel(int64_t* __restrict__ p, const int32_t* __restrict__ n_dev,
                                    int64_t per) {
  const int64_t n = int64_t(*n_dev) * per;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    p[i] = 0;
}

__global__ void subtract_kernel(const int64_t* __restrict__ parent,
                                const int64_t* __restrict__ built, int64_t* __restrict__ sibling,
                                int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(blockDim.x) * gridDim.x)
    sibling[i] = parent[i] - built[i];
}

// Grid: x = blocks of 256 words of one tile (word e = bin * 32 + within, as
// in the LDS image), y = tile, z strides over the jobs.  Each thread sums one
// word over the job's partial slots and writes the built and sibling values in
// the [feature][bin][g, h] layout.
__global__ __launch_bounds__(256) void hist_reduce_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs,
    int32_t n_jobs_host, const int32_t* __restrict__ n_jobs_dev, int32_t n_tiles,
    int32_t n_features, int32_t bin_stride, const long long* __restrict__ parent_base,
    long long* __restrict__ hist, int32_t accumulate) {
  const HistReduce j_first = int32_t(blockIdx.z) < n_jobs_host ? jobs[blockIdx.z] : HistReduce{};
  const int32_t n_jobs = n_jobs_dev ? *n_jobs_dev : n_jobs_host;
  const int n_words = bin_stride * 32;
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  const int within = e & 31, bin = e >> 5;
  const int f = t * kTile + (within & 15);
  if (e >= n_words || f >= n_features) return;  // no barriers below
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  const int64_t at = (int64_t(f) * bin_stride + bin) * 2 + (within >> 4);
  for (int32_t jb = blockIdx.z; jb < n_jobs; jb += gridDim.z) {
    const HistReduce j = jb == int32_t(blockIdx.z) ? j_first : jobs[jb];
    long long* built = hist + int64_t(j.slot) * node_elems + at;
    long long sum;
    if (j.nc == 1 && j.p0 < 0) {
      sum = *built;  // written directly by the node's only chunk
    } else {
      sum = sum_slots(partial + (int64_t(j.p0) * n_tiles + t) * n_words + e,
                      int64_t(n_tiles) * n_words, j.nc);
      if (accumulate) sum += *built;
      *built = sum;
    }
    if (j.sibling >= 0)
      hist[int64_t(j.sibling) * node_elems + at] = parent_base[j.parent + at] - sum;
  }
}

// One reduce job with many partial slots (a root pass: every chunk of the
// matrix): hist_reduce_kernel's sums with four times the loads in flight.
// Each 1024-thread workgroup takes 256 words of one tile; thread group q
// (256 threads) sums slots q, q + 4, ... of its word, and group 0 adds the
// four sums (exact in int64, so the order does not matter).
constexpr int kWideGroups = 4;
__global__ __launch_bounds__(256 * kWideGroups) void hist_reduce_wide_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs, int32_t n_tiles,
    int32_t n_features, int32_t bin_stride, const long long* __restrict__ parent_base,
    long long* __restrict__ hist, int32_t accumulate) {
  __shared__ long long part[kWideGroups - 1][256];
  const HistReduce j = jobs[0];
  const int q = threadIdx.x >> 8, t = threadIdx.x & 255;
  const int n_words = bin_stride * 32;
  const int e = blockIdx.x * 256 + t;
  const int tile = blockIdx.y;
  const int within = e & 31, bin = e >> 5;
  const int f = tile * kTile + (within & 15);
  const bool live = e < n_words && f < n_features;
  const bool direct = j.nc == 1 && j.p0 < 0;  // uniform: the node's only chunk wrote it
  long long sum = 0;
  if (live && !direct && q < j.nc) {
    const int32_t nq = (j.nc - q + kWideGroups - 1) / kWideGroups;  // slots q, q + 4, ...
    sum = sum_slots(partial + (int64_t(j.p0 + q) * n_tiles + tile) * n_words + e,
                    int64_t(kWideGroups) * n_tiles * n_words, nq);
  }
  if (q > 0) part[q - 1][t] = sum;
  __syncthreads();
  if (q > 0 || !live) return;  // no barriers below
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  const int64_t at = (int64_t(f) * bin_stride + bin) * 2 + (within >> 4);
  long long* built = hist + int64_t(j.slot) * node_elems + at;
  if (direct) {
    sum = *built;
  } else {
#pragma unroll
    for (int k = 0; k < kWideGroups - 1; ++k) sum += part[k][t];
    if (accumulate) sum += *built;
    *built = sum;
  }
  if (j.sibling >= 0) hist[int64_t(j.sibling) * node_elems + at] = parent_base[j.parent + at] - sum;
}

}  // namespace

void launch_fill_i64(int64_t* p, int64_t n, int64_t value, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_i64_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n, value);
  DP_HIP(hipGetLastError());
}

void launch_fill_u8(uint8_t* p, int64_t n, uint8_t value, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_u8_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n, value);
  DP_HIP(hipGetLastError());
}

void launch_iota_u32(uint32_t* p, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(iota_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, s, p, n);
  DP_HIP(hipGetLastError());
}

int32_t make_hist_work(const dp_bin_layout& layout, const int64_t* begin, const int64_t* end,
                       const int32_t* slots, int32_t n_nodes, bool allow_direct,
                       std::vector<HistWork>& work, std::vector<HistReduce>& jobs,
                       int32_t n_tiles, const HistConfig& cfg) {
  const int64_t T = n_tiles > 0 ? n_tiles : layout.n_tiles;
  const int64_t tpw = n_tiles > 0 ? 1 : cfg.tiles;  // present-value tiles: one per item
  const uint64_t pairs = n_tiles > 0 ? 0 : hist_pairs(layout.paired_tiles, cfg.tiles);
  if (pairs) check_pairs(layout);
  const int64_t G = hist_groups(int32_t(T), int32_t(tpw), pairs);  // work items per row chunk
  // About cfg.items items (two waves of resident workgroups on 256 CUs at the
  // default), at least kHistMinChunk rows each, so the per-item LDS clear and
  // store stay small.
  int64_t total = 0;
  for (int32_t i = 0; i < n_nodes; ++i) total += end[i] - begin[i];
  const int64_t chunk = hist_chunk(total, int32_t(G), cfg.items);
  struct Chunk {
    int32_t slot, partial;
    int64_t b, e;
  };
  std::vector<Chunk> chunks;
  jobs.clear();
  int32_t n_partial = 0;
  for (int32_t i = 0; i < n_nodes; ++i) {
    const int32_t slot = slots ? slots[i] : i;
    const int32_t nc = int32_t((end[i] - begin[i] + chunk - 1) / chunk);
    const bool direct = allow_direct && nc == 1;
    jobs.push_back({slot, -1, 0, direct ? -1 : n_partial, nc});
    for (int32_t k = 0; k < nc; ++k) {
      const int64_t b = begin[i] + k * chunk;
      chunks.push_back({slot, direct ? -1 : n_partial + k, b, std::min(b + chunk, end[i])});
    }
    if (!direct) n_partial += nc;
  }
  // Blocks are dispatched round-robin over the 8 XCDs (block id mod 8).  Item
  // order puts the tile groups of one row chunk on the same XCD in consecutive
  // dispatch slots, so that chunk's gradient pairs are read from HBM once and
  // then hit that XCD's L2.
  const int64_t groups = (int64_t(chunks.size()) + 7) / 8;
  work.assign(size_t(groups * G * 8), HistWork{0, 0, 0, 0, -1, 0});
  for (int64_t c = 0; c < int64_t(chunks.size()); ++c) {
    const Chunk& ch = chunks[size_t(c)];
    int64_t g = 0;  // tile group g: its first tile t
    for (int64_t t = 0; t < T; t += tpw) {
      if (pair_second(pairs, int32_t(t))) continue;
      const int64_t b = ((c / 8) * G + g) * 8 + (c % 8);
      work[size_t(b)] = {ch.slot, int32_t(t), ch.b, ch.e,
                         ch.partial < 0 ? -1 : int32_t(ch.partial * T + t), -1};
      ++g;
    }
  }
  return n_partial * int32_t(T);
}

uint64_t pair_tiles(const int32_t* n_bins, int32_t n_features, int32_t n_tiles, bool missing) {
  if (missing) return 0;
  auto narrow = [&](int32_t t) {  // every feature of tile t has at most 16 bins
    for (int32_t f = t * kTile; f < std::min((t + 1) * kTile, n_features); ++f)
      if (n_bins[f] > 16) return false;
    return true;
  };
  uint64_t m = 0;
  for (int32_t t = 0; t + 1 < n_tiles && t < 63;) {
    if (narrow(t) && narrow(t + 1)) {
      m |= 1ull << t;
      t += 2;
    } else {
      t += 1;
    }
  }
  return m;
}

void check_pairs(const dp_bin_layout& layout) {
  const uint64_t p = layout.paired_tiles;
  if (!p) return;
  need(layout.missing_bin < 0, "paired tiles need a matrix without missing values");
  need((p & (p << 1)) == 0, "a tile belongs to at most one pair");
  const int32_t last = std::min(layout.n_tiles - 1, 63);  // bit t needs tile t + 1
  need(last > 0 && (p >> last) == 0, "paired tile beyond the matrix");
}

namespace {
template <bool GATHER, int MODE, bool PAIRS = false>
auto hist_instance(const HistConfig& cfg) {
  if (cfg.deep)
    return cfg.tiles == 2
               ? (cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 2, 1, 0, true, PAIRS>
                                  : hist_kernel<GATHER, MODE, 2, 2, 0, true, PAIRS>)
               : (cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 1, 1, 0, true, PAIRS>
                                  : hist_kernel<GATHER, MODE, 1, 2, 0, true, PAIRS>);
  if (cfg.tiles == 2) {
    if (cfg.split == 4)
      return cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 2, 1, 4, false, PAIRS>
                             : hist_kernel<GATHER, MODE, 2, 2, 4, false, PAIRS>;
    if (cfg.split == 5)
      return cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 2, 1, 5, false, PAIRS>
                             : hist_kernel<GATHER, MODE, 2, 2, 5, false, PAIRS>;
    return cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 2, 1, 0, false, PAIRS>
                           : hist_kernel<GATHER, MODE, 2, 2, 0, false, PAIRS>;
  }
  return cfg.unroll == 1 ? hist_kernel<GATHER, MODE, 1, 1, 0, false, PAIRS>
                         : hist_kernel<GATHER, MODE, 1, 2, 0, false, PAIRS>;
}

// paired: the launch uses paired tiles (mode 0 only).
template <bool GATHER>
auto hist_mode(int mode, const HistConfig& cfg, bool paired) {
  if (paired) return hist_instance<GATHER, 0, true>(cfg);
  return mode == 1 ? hist_instance<GATHER, 1>(cfg)
                   : (mode == 2 ? hist_instance<GATHER, 2>(cfg) : hist_instance<GATHER, 0>(cfg));
}

// Raises the kernel's dynamic LDS limit when it needs more than the default
// 64 KiB, and returns how many of its workgroups one CU holds at once (LDS
// and registers); once per kernel.
int prepare_hist_kernel(const void* k, size_t lds) {
  static std::mutex lock;
  static std::vector<std::pair<const void*, int>> known;
  std::lock_guard<std::mutex> hold(lock);
  for (const auto& e : known)
    if (e.first == k) return e.second;
  if (lds > 65536)
    DP_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  int per_cu = 0;
  DP_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kHistThreads, lds));
  need(per_cu >= 1, "histogram kernel does not fit a CU");
  known.emplace_back(k, per_cu);
  return per_cu;
}

int device_cus() {
  static std::mutex lock;
  static int cached[64] = {};
  int dev = 0;
  DP_HIP(hipGetDevice(&dev));
  need(dev >= 0 && dev < 64, "device index out of range");
  std::lock_guard<std::mutex> hold(lock);
  if (cached[dev] == 0)
    DP_HIP(hipDeviceGetAttribute(&cached[dev], hipDeviceAttributeMultiprocessorCount, dev));
  return cached[dev];
}

int mode_of(bool missing, bool skip) { return missing ? 1 : (skip ? 2 : 0); }
}  // namespace

int hist_resident(bool gather, bool missing, bool skip, const HistConfig& cfg, bool paired) {
  const int mode = mode_of(missing, skip);
  need(!paired || mode == 0, "paired tiles take matrices without missing values or skip bins");
  auto kernel = gather ? hist_mode<true>(mode, cfg, paired) : hist_mode<false>(mode, cfg, paired);
  const size_t lds = size_t(cfg.tiles) * kLdsWords * sizeof(unsigned long long);
  return prepare_hist_kernel(reinterpret_cast<const void*>(kernel), lds) * device_cus();
}

void launch_hist(const uint8_t* bins, const dp_bin_layout& layout, const int32_t* gpair,
                 const uint32_t* ridx, const HistWork* work, int32_t n_work,
                 const int32_t* n_work_dev, int32_t bin_stride, int64_t* hist,
                 int64_t* partial, hipStream_t s, const uint8_t* row_major,
                 const HistConfig& cfg, const uint8_t* skip, bool fmaj) {
  if (n_work <= 0) return;
  need(bin_stride >= 1 && bin_stride <= kMaxBins, "histogram bin stride out of range");
  need(layout.tile_width == kTile, "histogram kernel needs 16-feature tiles");
  need((cfg.tiles == 1 || cfg.tiles == 2) && (cfg.unroll == 1 || cfg.unroll == 2) &&
           (cfg.split == 0 || cfg.split == 4 || cfg.split == 5) &&
           (cfg.deep == 0 || (cfg.deep == 1 && cfg.split == 0)),
       "histogram configuration out of range");
  auto* out = reinterpret_cast<unsigned long long*>(hist);
  auto* part = reinterpret_cast<unsigned long long*>(partial);
  const auto* gp = reinterpret_cast<const int2*>(gpair);
  // A missing value's byte 255 must not alias a real bin.
  if (layout.missing_bin >= 0) {
    need(layout.missing_bin == 255, "missing bin must be 255");
    need(bin_stride <= 255, "matrices with missing values have at most 255 bins");
  }
  const bool rows = ridx && row_major;
  const uint8_t* src = rows ? row_major : bins;
  const int64_t tile_step = rows ? kTile : layout.n_rows * kTile;
  const int64_t row_step = rows ? int64_t(layout.n_tiles) * kTile : kTile;
  // A pair's joint tile: tile n_tiles + k of the tile-major bins for the
  // layout's k-th pair, or in place of the pair's first tile in the row-major
  // copy (joint_first -1).
  const int32_t joint_first = rows ? -1 : layout.n_tiles;
  const bool missing = layout.missing_bin >= 0;
  need(!(missing && skip), "skip bins apply to matrices without missing values");
  const uint64_t pairs = hist_pairs(layout.paired_tiles, cfg.tiles);
  check_pairs(layout);
  need(!(pairs && skip), "paired tiles and skip bins do not combine");
  const int mode = mode_of(missing, skip != nullptr);
  auto kernel = ridx ? hist_mode<true>(mode, cfg, pairs != 0)
                     : hist_mode<false>(mode, cfg, pairs != 0);
  const size_t lds = size_t(cfg.tiles) * kLdsWords * sizeof(unsigned long long);
  // At most two rounds of resident workgroups; a multiple of 8.
  const int resident =
      prepare_hist_kernel(reinterpret_cast<const void*>(kernel), lds) * device_cus();
  int grid = n_work < 2 * resident ? n_work : 2 * resident;
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kHistThreads), lds, s, src, skip, layout.n_rows,
                     layout.n_features, layout.n_tiles, gp, ridx, work, n_work, n_work_dev,
                     bin_stride, out, part, tile_step, row_step, fmaj ? 1 : 0, pairs,
                     layout.paired_tiles, joint_first);
  DP_HIP(hipGetLastError());
}

void launch_zero_i64_dev(int64_t* p, const int32_t* n_dev, int64_t per, int64_t bound,
                         hipStream_t s) {
  if (bound <= 0 || per <= 0) return;
  hipLaunchKernelGGL(zero_i64_dev_kernel, dim3(grid_for(bound * per, 256, 8192)), dim3(256), 0, s,
                     p, n_dev, per);
  DP_HIP(hipGetLastError());
}

void launch_subtract(const int64_t* parent, const int64_t* built, int64_t* sibling, int64_t n,
                     hipStream_t s) {
  if (n <= 0) return;
  hipLaunchKernelGGL(subtract_kernel, dim3(grid_for(n, 256, 8192)), dim3(256), 0, s, parent,
                     built, sibling, n);
  DP_HIP(hipGetLastError());
}

void launch_hist_reduce(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                        const int32_t* n_jobs_dev, int32_t n_tiles, int32_t n_features,
                        int32_t bin_stride, const int64_t* parent_base, int64_t* hist,
                        bool accumulate, hipStream_t s) {
  if (n_jobs <= 0) return;
  need(bin_stride >= 1 && bin_stride <= kMaxBins, "histogram bin stride out of range");
  if (n_jobs == 1 && !n_jobs_dev) {  // one node (a root pass): the wide reduce
    hipLaunchKernelGGL(hist_reduce_wide_kernel,
                       dim3(unsigned(bin_stride * 32 + 255) / 256, unsigned(n_tiles)),
                       dim3(256 * kWideGroups), 0, s, reinterpret_cast<const long long*>(partial),
                       jobs, n_tiles, n_features, bin_stride,
                       reinterpret_cast<const long long*>(parent_base),
                       reinterpret_cast<long long*>(hist), accumulate ? 1 : 0);
    DP_HIP(hipGetLastError());
    return;
  }
  const dim3 grid(unsigned(bin_stride * 32 + 255) / 256, unsigned(n_tiles),
                  unsigned(n_jobs < 64 ? n_jobs : 64));
  hipLaunchKernelGGL(hist_reduce_kernel, grid, dim3(256), 0, s,
                     reinterpret_cast<const long long*>(partial), jobs, n_jobs, n_jobs_dev,
                     n_tiles, n_features, bin_stride,
                     reinterpret_cast<const long long*>(parent_base),
                     reinterpret_cast<long long*>(hist), accumulate ? 1 : 0);
  DP_HIP(hipGetLastError());
}

void launch_hist_sparse(const SparseBins& sp, int64_t n_rows, int32_t n_features,
                        const int32_t* gpair, const uint32_t* ridx, const HistWork* work,
                        int32_t n_work, const int32_t* n_work_dev, int32_t bin_stride,
                        int64_t* hist, int64_t* partial, hipStream_t s, const SparseEval* eval) {
  if (n_work <= 0) return;
  need(sp.n_tiles > 0, "present-value layout not built");
  need(bin_stride >= 1 && bin_stride <= kMaxBins, "histogram bin stride out of range");
  need(int64_t(sp.tile_features) * (bin_stride + 1) <= kSparsePlaneWords,
       "sparse tile exceeds its LDS plane");
  need(sp.bin_stride == bin_stride, "present-value entries were built for another bin stride");
  const size_t lds = size_t(kSparseLdsAlloc);  // two planes at fixed offsets
  SparseEvalArgs ev{};
  if (eval) {
    need(bin_stride <= 64, "evaluation in the present-value pass needs at most 64 bins");
    need(eval->parent_base && eval->n_bins && eval->node_sums && eval->exps && eval->cand,
         "evaluation in the present-value pass needs its inputs");
    const dp_train_param& q = eval->param;
    ev = SparseEvalArgs{reinterpret_cast<const long long*>(eval->parent_base), eval->n_bins,
                        reinterpret_cast<const long long*>(eval->node_sums), eval->exps,
                        Param{double(q.lambda), double(q.alpha), double(q.min_child_weight),
                              double(q.gamma)},
                        eval->fmask, eval->skip_bins, static_cast<FeatCand*>(eval->cand),
                        eval->store ? 1 : 0};
  }
  auto kernel = ridx ? (eval ? hist_sparse_kernel<true, true, kSparseEvalThreads>
                             : hist_sparse_kernel<true, false, kHistThreads>)
                     : (eval ? hist_sparse_kernel<false, true, kSparseEvalThreads>
                             : hist_sparse_kernel<false, false, kHistThreads>);
  static std::once_flag attr_once[4];
  std::call_once(attr_once[(ridx ? 1 : 0) + (eval ? 2 : 0)], [kernel] {
    DP_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(kSparseLdsAlloc)));
  });
  // Two workgroups per CU (at most 68 KiB of LDS each), a multiple of 8 for the XCD order.
  int grid = n_work < 1024 ? n_work : 1024;
  grid = (grid + 7) / 8 * 8;
  // Gathered rows read the row-major copy (when built), contiguous rows the
  // tile-major entries.
  const bool rows = ridx && sp.rptr.n > 0;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(eval ? kSparseEvalThreads : kHistThreads), lds, s,
                     rows ? sp.rptr.p : sp.ptr.p, rows ? sp.rentries.p : sp.entries.p,
                     n_rows, n_features, sp.tile_features, reinterpret_cast<const int2*>(gpair),
                     ridx, work, n_work, n_work_dev, bin_stride,
                     reinterpret_cast<unsigned long long*>(hist),
                     reinterpret_cast<unsigned long long*>(partial), ev,
                     rows ? sp.n_tiles : 1);
  DP_HIP(hipGetLastError());
}

void launch_hist_reduce_flat(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                             const int32_t* n_jobs_dev, int32_t n_tiles, int32_t tile_features,
                             int32_t n_features, int32_t bin_stride, const int64_t* parent_base,
                             int64_t* hist, hipStream_t s) {
  if (n_jobs <= 0) return;
  const int64_t words = int64_t(tile_features) * bin_stride * 2;
  const dim3 grid(unsigned((words + 255) / 256), unsigned(n_tiles),
                  unsigned(n_jobs < 64 ? n_jobs : 64));
  hipLaunchKernelGGL(hist_reduce_flat_kernel, grid, dim3(256), 0, s,
                     reinterpret_cast<const long long*>(partial), jobs, n_jobs, n_jobs_dev,
                     n_tiles, tile_features, n_features, bin_stride,
                     reinterpret_cast<const long long*>(parent_base),
                     reinterpret_cast<long long*>(hist));
  DP_HIP(hipGetLastError());
}

}  // namespace dp
