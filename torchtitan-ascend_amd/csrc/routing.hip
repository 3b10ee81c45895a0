// Routing kernels of the MoE expert path on MI355X (gfx950):
//   router top-k, per-expert histogram, stable counting sort (wavefront
//   ballot match + LDS wave prefixes), row gather (permute), gather-reduce
//   (unpermute / combine) and row dot products (routing-score gradients).
//
// Semantics follow the reference path:
//   * histogram + stable argsort of the flat expert labels: upstream
//     TorchTitan dispatch, reached from
//     torchtitanturbo/models/common/npu_gmm.py:106-108, and the index half of
//     torch_npu.npu_moe_token_permute (npu_permute.py:74-76);
//   * row gather = npu_moe_token_permute's row half / upstream dispatch's
//     `x[token_indices]` (+ fp32 score multiply when score_before_experts);
//   * gather-reduce = _npu_moe_token_unpermute_with_routing_map
//     (npu_permute.py:23-30) and upstream combine;
//   * unpermute grad = npu_moe_token_unpermute_with_routing_map_grad
//     (npu_permute.py:41-50).
// Every kernel that indexes memory with device-resident indices clamps them
// into the valid range, so a corrupt index array yields wrong values, never
// an out-of-bounds access.
#include <algorithm>
#include <mutex>

#include "../../include/ttamd_moe.h"
#include "common.h"
#include "gemm_common.h"
#include "kernels.h"

namespace ttamd {

// ---------------------------------------------------------------------------
// Stable counting sort.
//
// The flat label array is cut into chunks of kRouteChunk elements, one per
// workgroup.  Bucket E collects labels outside [0, E) so that every position
// of the output permutation is written exactly once.
//   pass 1 (hist): per-chunk bucket counts, stored bucket-major
//                  hist[b * nchunks + chunk];
//   pass 2 (scan): one workgroup turns hist into an exclusive prefix sum over
//                  that bucket-major order, which is exactly the first output
//                  position of (bucket b, chunk c);
//   pass 3 (rank): each wave owns 256 consecutive elements, finds equal
//                  labels among its 64 lanes with log2(E+1) ballots, and adds
//                  its wave-local rank to a per-wave running base kept in LDS.
// ---------------------------------------------------------------------------
constexpr int kRouteThreads = 256;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kRoutePerWave = 256;
constexpr int kRouteChunk = kRouteWaves * kRoutePerWave;  // 1024
constexpr int kScanThreads = 1024;
constexpr int kScanBatch = 16;  // histogram entries per scan thread loaded at once

template <typename IdxT>
__device__ __forceinline__ int bucket_of(const IdxT* labels, int i, int E) {
  const IdxT v = labels[i];
  return (v >= 0 && v < (IdxT)E) ? (int)v : E;
}

template <typename IdxT>
__global__ __launch_bounds__(kRouteThreads) void route_hist_kernel(
    const IdxT* __restrict__ labels, int M, int E, int nchunks,
    int* __restrict__ hist) {
  extern __shared__ int sh_hist[];  // E + 1
  for (int b = threadIdx.x; b <= E; b += kRouteThreads) sh_hist[b] = 0;
  __syncthreads();
  const int base = blockIdx.x * kRouteChunk;
  for (int i = threadIdx.x; i < kRouteChunk; i += kRouteThreads) {
    const int g = base + i;
    if (g < M) atomicAdd(&sh_hist[bucket_of(labels, g, E)], 1);
  }
  __syncthreads();
  for (int b = threadIdx.x; b <= E; b += kRouteThreads)
    hist[(size_t)b * nchunks + blockIdx.x] = sh_hist[b];
}

__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    int* __restrict__ hist, int n, int E, int nchunks, int M,
    int* __restrict__ counts, int* __restrict__ offsets) {
  extern __shared__ int sh_off[];  // E + 2
  __shared__ int wave_sums[kScanThreads / kWave];
  const int tid = threadIdx.x;
  if (n == 0) {  // no labels at all
    for (int e = tid; e <= E; e += kScanThreads) {
      if (offsets) offsets[e] = 0;
      if (e < E && counts) counts[e] = 0;
    }
    return;
  }
  const int per = (n + kScanThreads - 1) / kScanThreads;
  const int lo = min(tid * per, n);
  const int hi = min(lo + per, n);
  // A thread's segment is loaded as one batch of independent loads (up to
  // kScanBatch entries), not one dependent load per loop trip.
  int seg[kScanBatch];
  int s = 0;
  if (per <= kScanBatch) {
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) seg[j] = (lo + j < hi) ? hist[lo + j] : 0;
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) s += seg[j];
  } else {
    for (int i = lo; i < hi; ++i) s += hist[i];
  }
  const int incl = wave_inclusive_scan(s);
  const int w = tid / kWave, l = lane_id();
  if (l == kWave - 1) wave_sums[w] = incl;
  __syncthreads();
  if (w == 0) {
    const int v = (l < kScanThreads / kWave) ? wave_sums[l] : 0;
    const int vi = wave_inclusive_scan(v);
    if (l < kScanThreads / kWave) wave_sums[l] = vi - v;
  }
  __syncthreads();
  int run = wave_sums[w] + incl - s;
  if (per <= kScanBatch) {
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) {
      const int i = lo + j;
      if (i < hi) {
        hist[i] = run;
        if (i % nchunks == 0) sh_off[i / nchunks] = run;
        run += seg[j];
      }
    }
  } else {
    for (int i = lo; i < hi; ++i) {
      const int c = hist[i];
      hist[i] = run;
      if (i % nchunks == 0) sh_off[i / nchunks] = run;
      run += c;
    }
  }
  if (tid == 0) sh_off[E + 1] = M;
  __syncthreads();
  for (int e = tid; e <= E; e += kScanThreads) {
    if (offsets) offsets[e] = sh_off[e];
    if (e < E && counts) counts[e] = sh_off[e + 1] - sh_off[e];
  }
}

// Fused-scan form of the rank pass (FUSED = true): `base` is the raw
// per-chunk histogram, and every workgroup derives the first output position
// of (bucket b, its chunk c) itself,
//   base(b, c) = sum_{b' < b} total(b') + sum_{c' < c} hist[b][c'],
// reading the whole histogram (L2-resident; kFusedScanMax entries at most),
// which takes the single-workgroup scan launch off the path.  Workgroup 0
// then also writes counts / offsets, adds the counts to tokens_per_expert
// (the upstream router's load-balancing accumulator) and builds the grouped
// GEMMs' tile table of the expert-sorted rows, each when its pointer is set.
constexpr int kFusedScanMax = 32768;
constexpr int kBucketsPerThread = (1024 + 1 + kRouteThreads - 1) / kRouteThreads;  // E <= 1024
constexpr int kRowPrefetch = 64;  // chunk counts per bucket row loaded up front (FUSED, E < 256)

struct RouteExtras {
  int* counts;                // int32 [E]
  int* offsets;               // int32 [E + 1], exclusive
  float* tokens_per_expert;   // fp32 [E], += counts
  int4* plan_table;           // tile table (gemm_common.h block_tile_table)
  int* plan_count;
  int* plan_split_cnt;
  int plan_max_tiles;
  int plan_max_rows;
};

template <typename IdxT, bool FUSED>
__global__ __launch_bounds__(kRouteThreads) void route_rank_kernel(
    const IdxT* __restrict__ labels, const float* __restrict__ scores, int M,
    int E, int nbits, int nchunks, const int* __restrict__ base,
    int* __restrict__ sorted_idx, int* __restrict__ inverse,
    float* __restrict__ sorted_scores, const RouteExtras x) {
  // [kRouteWaves][E + 1] wave counters; FUSED: + chunk bases [E + 1],
  // bucket starts [E + 1] and kRouteWaves + 1 scan ints
  extern __shared__ int sh_cnt[];
  constexpr int NS = kRoutePerWave / kWave;
  const int E1 = E + 1;
  const int w = threadIdx.x / kWave, l = lane_id();
  const int wbase = blockIdx.x * kRouteChunk + w * kRoutePerWave;
  // Every global load of the pass is issued here, before the first LDS
  // wait, so that their latencies overlap: the wave's labels and scores and
  // (FUSED, one bucket row per thread) the row's first kRowPrefetch chunk
  // counts.
  // (Unconditional loads at clamped indices, M >= 1: a branch per load
  // would make the compiler wait for each before the next.)
  IdxT lab[NS];
  float scv[NS];
  const bool have_scores = sorted_scores != nullptr;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int gc = min(wbase + s * kWave + l, M - 1);
    lab[s] = labels[gc];
    scv[s] = have_scores ? scores[gc] : 0.f;
  }
  const int per = (E1 + kRouteThreads - 1) / kRouteThreads;
  // rows of a multiple of 4 counts are read as 16-byte vectors (the
  // histogram is 256-byte aligned)
  const bool row_pref = FUSED && per == 1 && nchunks <= kRowPrefetch && (nchunks & 3) == 0;
  int4 hv[FUSED ? kRowPrefetch / 4 : 1];
  if constexpr (FUSED) {
    const int4* row = (const int4*)(base + (size_t)threadIdx.x * nchunks);
    const bool have = row_pref && (int)threadIdx.x < E1;
#pragma unroll
    for (int c = 0; c < kRowPrefetch / 4; ++c) hv[c] = (have && 4 * c < nchunks) ? row[c] : make_int4(0, 0, 0, 0);
  }
  int bucket[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const IdxT v = lab[s];
    bucket[s] = (wbase + s * kWave + l < M) ? ((v >= 0 && v < (IdxT)E) ? (int)v : E) : 0;
  }
  for (int i = threadIdx.x; i < kRouteWaves * E1; i += kRouteThreads) sh_cnt[i] = 0;
  __syncthreads();

  uint64_t peers[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int g = wbase + s * kWave + l;
    const bool valid = g < M;
    const int b = bucket[s];
    uint64_t mask = ballot64(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool set = (b >> bit) & 1;
      const uint64_t bb = ballot64(set);
      mask &= set ? bb : ~bb;
    }
    peers[s] = mask;
    // One leader per distinct bucket of this step: no two lanes of the wave
    // touch the same counter, and other waves use their own row.
    if (valid && l == (int)__builtin_ctzll(mask))
      sh_cnt[w * E1 + b] += __builtin_popcountll(mask);
    lds_wait();  // the leader's counter update is visible to the next step
  }
  __syncthreads();
  int* sh_base = sh_cnt + kRouteWaves * E1;
  if constexpr (FUSED) {
    int* sh_start = sh_base + E1;
    int* sh_scan = sh_start + E1;
    // thread tid owns the consecutive buckets [tid * per, tid * per + per)
    const int tid = threadIdx.x;
    int tot[kBucketsPerThread], pre[kBucketsPerThread];
    int mine = 0;
#pragma unroll
    for (int i = 0; i < kBucketsPerThread; ++i) {
      const int b = tid * per + i;
      tot[i] = pre[i] = 0;
      if (row_pref) {
        if (i == 0) {
#pragma unroll
          for (int c = 0; c < kRowPrefetch / 4; ++c) {
            const int q[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              tot[0] += q[u];
              if (4 * c + u < (int)blockIdx.x) pre[0] += q[u];
            }
          }
        }
      } else if (i < per && b < E1) {
        const int* row = base + (size_t)b * nchunks;
        int c = 0;
        for (; c + 8 <= nchunks; c += 8) {
          int v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = row[c + u];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            tot[i] += v[u];
            if (c + u < (int)blockIdx.x) pre[i] += v[u];
          }
        }
        for (; c < nchunks; ++c) {
          const int v = row[c];
          tot[i] += v;
          if (c < (int)blockIdx.x) pre[i] += v;
        }
      }
      mine += tot[i];
    }
    // exclusive scan of the per-thread totals over the workgroup
    const int incl = wave_inclusive_scan(mine);
    if (l == kWave - 1) sh_scan[w] = incl;
    __syncthreads();
    if (tid == 0) {
      int run = 0;
      for (int ww = 0; ww < kRouteWaves; ++ww) {
        const int t = sh_scan[ww];
        sh_scan[ww] = run;
        run += t;
      }
    }
    __syncthreads();
    int start = sh_scan[w] + incl - mine;
#pragma unroll
    for (int i = 0; i < kBucketsPerThread; ++i) {
      const int b = tid * per + i;
      if (i < per && b < E1) {
        sh_start[b] = start;
        sh_base[b] = start + pre[i];
        if (blockIdx.x == 0) {
          if (x.offsets) x.offsets[b] = start;
          if (b < E) {
            if (x.counts) x.counts[b] = tot[i];
            if (x.tokens_per_expert) x.tokens_per_expert[b] += (float)tot[i];
          }
        }
        start += tot[i];
      }
    }
    __syncthreads();
    if (blockIdx.x == 0 && x.plan_table) {
      auto range = [&](int e, int& r0, int& r1) {
        r0 = sh_start[e];
        r1 = sh_start[e + 1];
      };
      block_tile_table<kRouteThreads>(range, E, x.plan_max_tiles, x.plan_max_rows, x.plan_table, x.plan_count,
                                      x.plan_split_cnt, sh_scan);
    }
  }
  // Running base of (wave w, bucket b) = chunk base + counts of earlier waves.
  for (int b = threadIdx.x; b < E1; b += kRouteThreads) {
    int run = FUSED ? sh_base[b] : base[(size_t)b * nchunks + blockIdx.x];
#pragma unroll
    for (int ww = 0; ww < kRouteWaves; ++ww) {
      const int t = sh_cnt[ww * E1 + b];
      sh_cnt[ww * E1 + b] = run;
      run += t;
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < kRoutePerWave / kWave; ++s) {
    const int g = wbase + s * kWave + l;
    const bool valid = g < M;
    const int b = bucket[s];
    const uint64_t mask = peers[s];
    int pos = 0;
    if (valid) pos = sh_cnt[w * E1 + b] + __builtin_popcountll(mask & lanemask_lt());
    lds_wait();  // every lane has read the counter before its leader updates it
    if (valid && l == (int)__builtin_ctzll(mask))
      sh_cnt[w * E1 + b] += __builtin_popcountll(mask);
    lds_wait();  // the leader's counter update is visible to the next step
    if (valid) {
      pos = min(max(pos, 0), M - 1);
      sorted_idx[pos] = g;
      if (inverse) inverse[g] = pos;
      if (sorted_scores) sorted_scores[pos] = scv[s];
    }
  }
}

size_t route_hist_bytes(int64_t M, int E) {
  const int64_t nchunks = (M + kRouteChunk - 1) / kRouteChunk;
  return (size_t)((E + 1) * nchunks) * sizeof(int);
}

size_t route_workspace_bytes(int64_t M, int E) { return route_hist_bytes(M, E) + 256; }

// ---------------------------------------------------------------------------
// Library-owned route workspace (the allocation-free entry point).
//
// `scratch` is a file-scope device array: every device the library runs on
// holds its own copy, at its own address, from the moment the code object is
// loaded there until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host that name is a stand-in, not a device
// address): the address of each device's copy is looked up once per device
// with hipGetSymbolAddress, with that device current, and cached here.
// ---------------------------------------------------------------------------
constexpr size_t kRouteScratchBytes = TTAMD_ROUTE_NOALLOC_WORKSPACE_BYTES;
static __device__ __align__(256) int scratch[kRouteScratchBytes / sizeof(int)];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

size_t route_scratch_bytes() { return kRouteScratchBytes; }

hipError_t route_scratch(hipStream_t stream, void** ptr) {
  *ptr = nullptr;
  int dev = 0;
  hipError_t err = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int prev = 0;
    err = hipGetDevice(&prev);
    if (err != hipSuccess) return err;
    if (prev != dev && (err = hipSetDevice(dev)) != hipSuccess) return err;
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev != dev) {
      const hipError_t back = hipSetDevice(prev);
      if (err == hipSuccess) err = back;
    }
    if (err != hipSuccess) return err;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

// counts of the route (after its scan) added into tokens_per_expert
__global__ __launch_bounds__(256) void accumulate_counts_kernel(const int* __restrict__ counts, int E,
                                                                float* __restrict__ acc) {
  for (int e = blockIdx.x * 256 + threadIdx.x; e < E; e += gridDim.x * 256) acc[e] += (float)counts[e];
}

namespace {

int route_nbits(int E) {
  int nbits = 0;
  while ((1 << nbits) <= E) ++nbits;  // bucket values 0..E
  return nbits;
}

template <bool FUSED>
hipError_t launch_rank(const void* labels, bool is64, const float* scores, int M, int E, int nchunks,
                       const int* hist, int* sorted_idx, int* inverse, float* sorted_scores,
                       const RouteExtras& x, hipStream_t stream) {
  const size_t sh = ((size_t)(kRouteWaves + (FUSED ? 2 : 0)) * (E + 1) + (FUSED ? kRouteWaves + 1 : 0)) *
                    sizeof(int);
  const int nbits = route_nbits(E);
  if (is64)
    return launch_k(false, route_rank_kernel<int64_t, FUSED>, dim3(nchunks), dim3(kRouteThreads), (uint32_t)sh,
                    stream, (const int64_t*)labels, scores, M, E, nbits, nchunks, hist, sorted_idx, inverse,
                    sorted_scores, x);
  return launch_k(false, route_rank_kernel<int32_t, FUSED>, dim3(nchunks), dim3(kRouteThreads), (uint32_t)sh,
                  stream, (const int32_t*)labels, scores, M, E, nbits, nchunks, hist, sorted_idx, inverse,
                  sorted_scores, x);
}

}  // namespace

bool route_fused_scan(int64_t M, int E) {
  const int64_t nchunks = (M + kRouteChunk - 1) / kRouteChunk;
  return (int64_t)(E + 1) * nchunks <= kFusedScanMax;
}

int route_num_chunks(int64_t M) { return (int)((M + kRouteChunk - 1) / kRouteChunk); }

int route_chunk_labels() { return kRouteChunk; }

hipError_t launch_route_from_hist(const void* labels, bool is64, int M, int E, const float* scores,
                                  int* counts, int* offsets, int* sorted_idx, int* inverse,
                                  float* sorted_scores, int* hist, float* tokens_per_expert,
                                  void* plan, int plan_max_rows, hipStream_t stream) {
  const int nchunks = route_num_chunks(M);
  RouteExtras x = {};
  x.counts = counts;
  x.offsets = offsets;
  x.tokens_per_expert = tokens_per_expert;
  if (plan) {
    const TileTable tt = tile_table_in(plan);
    x.plan_table = tt.table;
    x.plan_count = tt.count;
    x.plan_split_cnt = tt.split_cnt;
    x.plan_max_tiles = max_row_tiles(M, E);
    x.plan_max_rows = plan_max_rows;
  }
  if (M == 0) {  // nothing routed: zero counts / offsets, an empty tile table
    hipError_t err = launch_k(false, route_scan_kernel, dim3(1), dim3(kScanThreads),
                              (uint32_t)((E + 2) * sizeof(int)), stream, hist, 0, E, 1, 0, counts, offsets);
    if (err == hipSuccess && plan) err = launch_tile_map(offsets + 1, E, 0, plan_max_rows, plan, stream);
    return err;
  }
  if (route_fused_scan(M, E))
    return launch_rank<true>(labels, is64, scores, M, E, nchunks, hist, sorted_idx, inverse, sorted_scores, x,
                             stream);
  // large histograms: the single-workgroup scan, then the rank pass, the
  // tile table and the accumulation as separate launches
  hipError_t err = launch_k(false, route_scan_kernel, dim3(1), dim3(kScanThreads), (uint32_t)((E + 2) * sizeof(int)),
                            stream, hist, (E + 1) * nchunks, E, nchunks, M, counts, offsets);
  if (err == hipSuccess) err = launch_rank<false>(labels, is64, scores, M, E, nchunks, hist, sorted_idx, inverse,
                                      sorted_scores, RouteExtras{}, stream);
  if (err == hipSuccess && plan) err = launch_tile_map(offsets + 1, E, M, plan_max_rows, plan, stream);
  if (err == hipSuccess && tokens_per_expert) {
    err = launch_k(false, accumulate_counts_kernel, dim3((E + 255) / 256), dim3(256), 0, stream, counts, E,
                   tokens_per_expert);
  }
  return err;
}

hipError_t launch_route(const void* labels, bool is64, int M, int E,
                        const float* scores, int* counts, int* offsets,
                        int* sorted_idx, int* inverse, float* sorted_scores,
                        void* ws, hipStream_t stream) {
  const int nchunks = route_num_chunks(M);
  int* hist = (int*)ws;
  if (M > 0) {
    const size_t sh1 = (size_t)(E + 1) * sizeof(int);
    hipError_t err =
        is64 ? launch_k(false, route_hist_kernel<int64_t>, dim3(nchunks), dim3(kRouteThreads), (uint32_t)sh1, stream,
                        (const int64_t*)labels, M, E, nchunks, hist)
             : launch_k(false, route_hist_kernel<int32_t>, dim3(nchunks), dim3(kRouteThreads), (uint32_t)sh1, stream,
                        (const int32_t*)labels, M, E, nchunks, hist);
    if (err != hipSuccess) return err;
  }
  return launch_route_from_hist(labels, is64, M, E, scores, counts, offsets, sorted_idx, inverse, sorted_scores,
                                hist, nullptr, nullptr, 0, stream);
}

// ---------------------------------------------------------------------------
// Row movement.  Rows are moved as 16-byte chunks (8 bf16).
// ---------------------------------------------------------------------------
constexpr int kMoveThreads = 256;

// out[r] = in[clamp(src[r] / div)] * (scale ? scale[scale_by_src ? src[r] : r] : 1)
// One wave per output row (grid-stride over rows): the source row id and
// scale are read once per row, then the row moves in batches of
// kGatherUnroll 16-byte chunks per lane, every load of a batch issued before
// its stores.  Both the read and the write of a row are contiguous and
// streaming (non-temporal): C4's regroup 199 -> 189 us.  (The scatter-form
// dispatch below keeps cached stores: its K copies per row were slower as
// streaming writes, C2 49 -> 57 us.)
constexpr int kGatherUnroll = 8;

__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint4* __restrict__ in, const int* __restrict__ src,
    const float* __restrict__ scale, int scale_by_src, int n_in, int n_src_max,
    int rows, int cpr, int div, uint4* __restrict__ out) {
  const int nw = gridDim.x * 4;
  const int l = lane_id();
  for (int r = blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += nw) {
    int s = src ? src[r] : r;
    s = min(max(s, 0), n_src_max - 1);
    const int srow = min(s / div, n_in - 1);
    const float sc = scale ? scale[scale_by_src ? s : r] : 1.f;
    const uint4* irow = in + (int64_t)srow * cpr;
    uint4* orow = out + (int64_t)r * cpr;
    for (int c0 = 0; c0 < cpr; c0 += 64 * kGatherUnroll) {
      uint4 v[kGatherUnroll];
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) {
        const int c = c0 + 64 * u + l;
        if (c < cpr) v[u] = load_stream(&irow[c]);
      }
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) {
        const int c = c0 + 64 * u + l;
        if (c < cpr) {
          uint4 o = v[u];
          if (scale) {
            float f[8];
            unpack8(o, f);
#pragma unroll
            for (int i = 0; i < 8; ++i) f[i] *= sc;
            o = pack8(f);
          }
          store_stream(&orow[c], o);
        }
      }
    }
  }
}

hipError_t launch_gather_rows(const void* in, const int* src, const float* scale,
                              bool scale_by_src, int n_in, int n_src_max, int rows,
                              int hidden, int div, void* out, hipStream_t stream) {
  const int cpr = hidden / 8;
  if ((int64_t)rows * cpr == 0) return hipSuccess;
  const int grid = (int)std::min<int64_t>(((int64_t)rows + 3) / 4, 2048);
  return launch_k(false, gather_rows_kernel, dim3(grid), dim3(256), 0, stream, (const uint4*)in, src, scale,
                  scale_by_src ? 1 : 0, n_in, n_src_max, rows, cpr, div, (uint4*)out);
}

// Dispatch in scatter form: one wave per token reads its row once and writes
// the top-k copies, out[inverse[t*K + k]] = x[t] (* scores[t*K + k], rounded
// to bf16 once).  The same rows as gather_rows with src = sorted order, but x
// is read once from HBM instead of K times through the caches.
constexpr int kDispatchUnroll = 4;

__global__ __launch_bounds__(256) void dispatch_rows_kernel(const uint4* __restrict__ in,
                                                            const int* __restrict__ inverse,
                                                            const float* __restrict__ scores, int T,
                                                            int K, int cpr, int M,
                                                            uint4* __restrict__ out) {
  const int nw = gridDim.x * 4;
  const int l = threadIdx.x & 63;
  for (int t = blockIdx.x * 4 + (threadIdx.x >> 6); t < T; t += nw) {
    int dst = 0;
    float sc = 1.f;
    if (l < K) {
      dst = min(max(inverse[(int64_t)t * K + l], 0), M - 1);
      if (scores) sc = scores[(int64_t)t * K + l];
    }
    const uint4* irow = in + (int64_t)t * cpr;
    for (int c0 = 0; c0 < cpr; c0 += 64 * kDispatchUnroll) {
      uint4 v[kDispatchUnroll];
#pragma unroll
      for (int u = 0; u < kDispatchUnroll; ++u) {
        const int c = c0 + 64 * u + l;
        if (c < cpr) v[u] = irow[c];
      }
      for (int k = 0; k < K; ++k) {
        const int d = __shfl(dst, k, 64);
        const float s = __shfl(sc, k, 64);
        uint4* orow = out + (int64_t)d * cpr;
#pragma unroll
        for (int u = 0; u < kDispatchUnroll; ++u) {
          const int c = c0 + 64 * u + l;
          if (c < cpr) {
            uint4 o = v[u];
            if (scores) {
              float f[8];
              unpack8(o, f);
#pragma unroll
              for (int i = 0; i < 8; ++i) f[i] *= s;
              o = pack8(f);
            }
            orow[c] = o;
          }
        }
      }
    }
  }
}

hipError_t launch_dispatch_rows(const void* in, const int* inverse, const float* scores, int T, int K,
                                int hidden, void* out, hipStream_t stream) {
  if ((int64_t)T * K == 0) return hipSuccess;
  const int cpr = hidden / 8;
  const int grid = (int)std::min<int64_t>(((int64_t)T + 3) / 4, 2048);
  return launch_k(false, dispatch_rows_kernel, dim3(grid), dim3(256), 0, stream, (const uint4*)in, inverse,
                  scores, T, K, cpr, T * K, (uint4*)out);
}

// inv[sorted[j]] = j.
__global__ __launch_bounds__(kMoveThreads) void invert_perm_kernel(
    const int* __restrict__ sorted, int M, int* __restrict__ inv) {
  for (int j = blockIdx.x * kMoveThreads + threadIdx.x; j < M; j += gridDim.x * kMoveThreads) {
    const int s = min(max(sorted[j], 0), M - 1);
    inv[s] = j;
  }
}

hipError_t launch_invert_perm(const int* sorted, int M, int* inv, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  int g = (M + kMoveThreads - 1) / kMoveThreads;
  if (g > 4096) g = 4096;
  return launch_k(false, invert_perm_kernel, dim3(g), dim3(kMoveThreads), 0, stream, sorted, M, inv);
}

// out[t] = sum_k w(t,k) * in[j(t,k)],  j = inverse ? inverse[t*topk+k] : t*topk+k.
// The K rows of a chunk are loaded kCombineBatch at a time, all loads of a
// batch issued before any of them is used, so a thread keeps up to
// kCombineBatch 16-byte loads in flight; the sum runs in k order.  The
// routed rows are read once and the output written once, both as streaming
// (non-temporal) accesses: they then do not allocate in L2, where they
// would evict (and force the write-back of) the dirty lines the w2 GEMM
// leaves behind (C2: 54 -> 48 us in the layer step).
constexpr int kCombineBatch = 8;

__global__ __launch_bounds__(kMoveThreads) void combine_kernel(
    const uint4* __restrict__ in, const int* __restrict__ inverse,
    const float* __restrict__ probs, int T, int topk, int M, int cpr,
    uint4* __restrict__ out) {
  const int total = T * cpr;
  const int stride = gridDim.x * kMoveThreads;
  for (int idx = blockIdx.x * kMoveThreads + threadIdx.x; idx < total; idx += stride) {
    const int t = idx / cpr;
    const int c = idx - t * cpr;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < topk; k0 += kCombineBatch) {
      uint4 v[kCombineBatch];
      float w[kCombineBatch];
#pragma unroll
      for (int b = 0; b < kCombineBatch; ++b) {
        const int k = k0 + b;
        if (k < topk) {
          const int s = t * topk + k;
          int j = inverse ? inverse[s] : s;
          j = min(max(j, 0), M - 1);
          w[b] = probs ? probs[s] : 1.f;
          v[b] = load_stream(&in[(size_t)j * cpr + c]);
        }
      }
#pragma unroll
      for (int b = 0; b < kCombineBatch; ++b) {
        if (k0 + b < topk) {
          float f[8];
          unpack8(v[b], f);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += w[b] * f[i];
        }
      }
    }
    store_stream(&out[idx], pack8(acc));
  }
}

hipError_t launch_combine(const void* in, const int* inverse, const float* probs, int T,
                          int topk, int hidden, void* out, hipStream_t stream) {
  const int cpr = hidden / 8;
  const int64_t total = (int64_t)T * cpr;
  if (total == 0) return hipSuccess;
  int64_t g = (total + kMoveThreads - 1) / kMoveThreads;
  if (g > 8192) g = 8192;
  return launch_k(false, combine_kernel, dim3((int)g), dim3(kMoveThreads), 0, stream, (const uint4*)in, inverse,
                  probs, T, topk, T * topk, cpr, (uint4*)out);
}

// out[o(j)] = <a[j], b[clamp(bidx[j] / bdiv)]>, o(j) = out_by_bidx ? bidx[j] : j.
__global__ __launch_bounds__(kMoveThreads) void rowdot_kernel(
    const uint4* __restrict__ a, const uint4* __restrict__ b, const int* __restrict__ bidx,
    int bdiv, int out_by_bidx, int rows, int n_b, int n_out, int cpr,
    float* __restrict__ out) {
  const int wave = (blockIdx.x * kMoveThreads + threadIdx.x) / kWave;
  const int nwaves = gridDim.x * kMoveThreads / kWave;
  const int l = lane_id();
  for (int j = wave; j < rows; j += nwaves) {
    int s = bidx ? bidx[j] : j;
    const int sb = min(max(s / bdiv, 0), n_b - 1);
    float acc = 0.f;
    for (int c = l; c < cpr; c += kWave) {
      float fa[8], fb[8];
      unpack8(a[(size_t)j * cpr + c], fa);
      unpack8(b[(size_t)sb * cpr + c], fb);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += fa[i] * fb[i];
    }
    acc = wave_reduce_sumf(acc);
    if (l == 0) {
      const int o = out_by_bidx ? min(max(s, 0), n_out - 1) : j;
      out[o] = acc;
    }
  }
}

hipError_t launch_rowdot(const void* a, const void* b, const int* bidx, int bdiv,
                         bool out_by_bidx, int rows, int n_b, int n_out, int hidden,
                         float* out, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  int64_t g = ((int64_t)rows * kWave + kMoveThreads - 1) / kMoveThreads;
  if (g > 8192) g = 8192;
  return launch_k(false, rowdot_kernel, dim3((int)g), dim3(kMoveThreads), 0, stream, (const uint4*)a,
                  (const uint4*)b, bidx, bdiv, out_by_bidx ? 1 : 0, rows, n_b, n_out, hidden / 8, out);
}

// ---------------------------------------------------------------------------
// Regroup labels: rows arrive as G consecutive groups (rank r, expert e),
// g = r * E_loc + e; label = g % E_loc.  Each block scans the G counts in
// LDS and binary-searches the group of each of its rows.
// ---------------------------------------------------------------------------
constexpr int kLabelMaxGroups = 8192;

__global__ __launch_bounds__(kMoveThreads) void group_labels_kernel(
    const int* __restrict__ counts, int G, int E_loc, int rows, int* __restrict__ labels) {
  __shared__ int incl[kLabelMaxGroups];
  __shared__ int wave_sums[kMoveThreads / kWave];
  const int tid = threadIdx.x;
  const int per = (G + kMoveThreads - 1) / kMoveThreads;
  const int lo = min(tid * per, G), hi = min(lo + per, G);
  int s = 0;
  for (int i = lo; i < hi; ++i) s += max(counts[i], 0);
  const int in = wave_inclusive_scan(s);
  const int w = tid / kWave, l = lane_id();
  if (l == kWave - 1) wave_sums[w] = in;
  __syncthreads();
  int base = 0;
  for (int ww = 0; ww < w; ++ww) base += wave_sums[ww];
  int run = base + in - s;
  for (int i = lo; i < hi; ++i) {
    run += max(counts[i], 0);
    incl[i] = run;
  }
  __syncthreads();
  const int total = incl[G - 1];
  for (int j = blockIdx.x * kMoveThreads + tid; j < rows; j += gridDim.x * kMoveThreads) {
    int lab = E_loc;
    if (j < total) {
      int a = 0, b = G - 1;  // first g with incl[g] > j
      while (a < b) {
        const int m = (a + b) >> 1;
        if (incl[m] > j) b = m; else a = m + 1;
      }
      lab = a % E_loc;
    }
    labels[j] = lab;
  }
}

hipError_t launch_group_labels(const int* counts_group, int G, int E_loc, int rows, int* labels,
                               hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  int g = (rows + kMoveThreads - 1) / kMoveThreads;
  if (g > 1024) g = 1024;
  return launch_k(false, group_labels_kernel, dim3(g), dim3(kMoveThreads), 0, stream, counts_group, G, E_loc,
                  rows, labels);
}

// ---------------------------------------------------------------------------
// Router top-k: one wave per token.  Each lane holds ceil(E/64) scores in
// registers; k rounds of a wave-wide argmax of the selection keys (sel_key:
// NaN first, then value desc, -inf after every finite value), ties to the
// lower expert id.
// ---------------------------------------------------------------------------
constexpr int kTopkMaxPerLane = 16;  // E <= 1024

template <int PER_LANE>
__global__ __launch_bounds__(kMoveThreads) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int K,
    int score_func, int renorm, float renorm_eps, float route_scale,
    float* __restrict__ top_scores, int64_t* __restrict__ top_idx) {
  const int wave = (blockIdx.x * kMoveThreads + threadIdx.x) / kWave;
  const int nwaves = gridDim.x * kMoveThreads / kWave;
  const int l = lane_id();
  for (int t = wave; t < T; t += nwaves) {
    const float* row = logits + (size_t)t * E;
    float sc[PER_LANE];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) {
      const int e = i * kWave + l;
      sc[i] = (e < E) ? row[e] : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    if (score_func == 0) {  // softmax in fp32
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i) {
        const int e = i * kWave + l;
        sc[i] = (e < E) ? expf(sc[i] - mx) : 0.f;
        sum += sc[i];
      }
      sum = wave_reduce_sumf(sum);
      const float inv = 1.f / sum;
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i) sc[i] = sc[i] * inv;
    } else {  // sigmoid
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i) sc[i] = 1.f / (1.f + expf(-sc[i]));
    }
    // selection keys (sel_key: NaN first, then value desc, -inf after every
    // finite value; 0 = not pickable)
    uint32_t key[PER_LANE];
#pragma unroll
    for (int i = 0; i < PER_LANE; ++i) {
      const int e = i * kWave + l;
      key[i] = (e < E) ? sel_key(bias ? sc[i] + bias[e] : sc[i]) : 0u;
    }
    float picked_sum = 0.f;
    float my_val = 0.f;
    int my_idx = 0;
    for (int k = 0; k < K; ++k) {
      // lane-local best (key desc, index asc)
      uint32_t bk = 0u;
      int bi = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i) {
        const int e = i * kWave + l;
        if (key[i] > bk) {  // slots in increasing e: the first maximum is the lowest id
          bk = key[i];
          bi = e;
        }
      }
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) {
        const uint32_t ok = (uint32_t)__shfl_xor((int)bk, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ok > bk || (ok == bk && oi < bi)) {
          bk = ok;
          bi = oi;
        }
      }
      // bi is wave-uniform now; fetch its unbiased score from its owner lane.
      const int owner = bi & (kWave - 1);
      const int slot = bi / kWave;
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i)
        if (i == slot) v = sc[i];
      v = __shfl(v, owner, kWave);
#pragma unroll
      for (int i = 0; i < PER_LANE; ++i)
        if (i == slot && l == owner) key[i] = 0u;
      if (bi >= E) bi = 0;  // unreachable when K <= E; keeps the index in range
      picked_sum += v;
      if (l == k) {
        my_val = v;
        my_idx = bi;
      }
    }
    if (l < K) {
      float v = my_val;
      if (renorm) v = v / (picked_sum + renorm_eps);
      v *= route_scale;
      top_scores[(size_t)t * K + l] = v;
      top_idx[(size_t)t * K + l] = my_idx;
    }
  }
}

hipError_t launch_router_topk(const float* logits, const float* bias, int T, int E, int K,
                              int score_func, int renorm, float renorm_eps, float route_scale,
                              float* top_scores, int64_t* top_idx, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  int64_t g = ((int64_t)T * kWave + kMoveThreads - 1) / kMoveThreads;
  if (g > 8192) g = 8192;
  const int per = (E + kWave - 1) / kWave;
  auto go = [&](auto kernel) {
    return launch_k(false, kernel, dim3((int)g), dim3(kMoveThreads), 0, stream, logits, bias, T, E, K, score_func,
                    renorm, renorm_eps, route_scale, top_scores, top_idx);
  };
  if (per <= 1) return go(router_topk_kernel<1>);
  if (per <= 2) return go(router_topk_kernel<2>);
  if (per <= 4) return go(router_topk_kernel<4>);
  if (per <= 8) return go(router_topk_kernel<8>);
  return go(router_topk_kernel<kTopkMaxPerLane>);
}

}  // namespace ttamd
