// Device-wide scan and stable LSD radix sort building blocks (256-thread blocks = 4 wave64s).
//
// Radix sort pass = three kernels:
//   upsweep   : per-block digit histograms, stored digit-major hist[d * nb + b]
//   scan_hist : one block per digit, exclusive scan over blocks + digit totals
//   downsweep : per block, wave-private ranking of contiguous segments (wave64 ballot match),
//               then an LDS reorder by digit and coalesced stores of each digit's run.
#pragma once
#include "xsg_common.h"

namespace xsg {

constexpr int kSortBlock = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortBlock * kSortItems;  // keys per block and pass
constexpr int kRadix = 256;
constexpr int kWaves = kSortBlock / 64;

template <int ITEMS = kSortItems>
inline unsigned sort_blocks(int64_t n) {
    return (unsigned)((n + kSortBlock * ITEMS - 1) / (kSortBlock * ITEMS));
}

template <typename T>
XSG_DEV T wave_inclusive_scan(T v) {
    const int lane = __lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const T t = __shfl_up(v, off, 64);
        if (lane >= off) v += t;
    }
    return v;
}

// Exclusive scan over the 256 threads of a block; `lds` holds kWaves elements.
template <typename T>
XSG_DEV T block_exclusive_scan(T v, T* lds, T& total) {
    const T inc = wave_inclusive_scan(v);
    const int wave = threadIdx.x >> 6;
    if (__lane_id() == 63) lds[wave] = inc;
    __syncthreads();
    T before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const T x = lds[w];
        if (w < wave) before += x;
        tot += x;
    }
    __syncthreads();
    total = tot;
    return before + inc - v;
}

template <typename T>
XSG_DEV T block_reduce_sum(T v, T* lds) {
    T total;
    block_exclusive_scan(v, lds, total);
    return total;
}

// ---------------------------------------------------------------- radix sort passes
template <typename K>
XSG_DEV uint32_t digit_of(K key, int shift, int bits) {
    return (uint32_t)((key >> shift) & (K)((1u << bits) - 1u));
}

// The most significant RB bits of a 32-bit key's offset from the smallest key: the digit of a
// most-significant-digit pass that splits the keys into 1 << RB buckets of consecutive key values.
// The key range comes from the device as n_part partial ranges (smallest, largest) in `range`, each
// (~0, 0) when it saw no key. shift: the bits below the digit.
struct KeyRange {
    uint32_t kmin;
    int shift;
};
XSG_DEV KeyRange key_range(const uint32_t* __restrict__ range, int n_part, int rb) {
    uint32_t kmin = 0xffffffffu, kmax = 0u;
    for (int i = 0; i < n_part; ++i) {
        kmin = min(kmin, range[2 * i]);
        kmax = max(kmax, range[2 * i + 1]);
    }
    const uint32_t span = kmax > kmin ? kmax - kmin : 0u;  // kmin > kmax: no keys
    const int width = span ? 32 - __clz(span) : 0;
    return KeyRange{kmin, max(0, width - rb)};
}

// a pass's digit: bits [shift, shift + bits) of the key, or with a key range the top digit of the
// key's offset in the range
template <typename K, bool RANGE>
XSG_DEV uint32_t pass_digit(K key, int shift, int bits, const KeyRange& kr) {
    if constexpr (RANGE) return (uint32_t)(((uint32_t)key - kr.kmin) >> kr.shift) & ((1u << bits) - 1u);
    else return digit_of<K>(key, shift, bits);
}

// A tile is kSortBlock * ITEMS keys; the tiles holding keys are [0, ceil(n / tile)). n_dev
// (optional): the element count read on the device, at most n, with the grid sized on the host for
// n: the upsweep and downsweep workgroups then loop over the tiles (grid stride), so that a grid
// smaller than n's tile count can serve a count that is usually far below n.
template <int ITEMS>
XSG_DEV unsigned active_tiles(int64_t n, const uint32_t* n_dev) {
    if (n_dev) n = min(n, (int64_t)*n_dev);
    return (unsigned)((n + kSortBlock * ITEMS - 1) / (kSortBlock * ITEMS));
}

// The tiles a grid-striding pass visits: with at least 8 workgroups each XCD (workgroups are dispatched
// round-robin over the 8 XCDs) takes a contiguous eighth of the tiles, so that neighbouring tiles'
// histogram words, consecutive in each digit's row, meet in one L2; smaller grids stride plainly.
struct TileWalk {
    unsigned t, end, step;
};
XSG_DEV TileWalk tile_walk(unsigned nt) {
    const unsigned g = gridDim.x;
    if (g < 8u) return TileWalk{blockIdx.x, nt, g};
    const unsigned x = blockIdx.x & 7u, r = blockIdx.x >> 3;
    const unsigned t0 = (unsigned)((uint64_t)nt * x / 8u), t1 = (unsigned)((uint64_t)nt * (x + 1u) / 8u);
    return TileWalk{t0 + r, t1, (g - x + 7u) >> 3};  // the XCD's workgroups: ceil((g - x) / 8)
}

// RB: bits per digit (8 by default; up to 10 for a single pass over a wider key, the digit-indexed
// arrays then holding 1 << RB entries, R / kSortBlock per thread).
template <typename K, int ITEMS = kSortItems, int RB = 8, bool RANGE = false>
__global__ __launch_bounds__(kSortBlock) void radix_upsweep(const K* __restrict__ keys, int64_t n, int shift,
                                                            int bits, uint32_t* __restrict__ hist, unsigned nb,
                                                            const uint32_t* __restrict__ n_dev,
                                                            const uint32_t* __restrict__ range = nullptr,
                                                            int range_parts = 0) {
    constexpr int R = 1 << RB, DPT = R / kSortBlock;
    static_assert(DPT >= 1 && DPT * kSortBlock == R, "a digit count that is a multiple of the block");
    if (n_dev) n = min(n, (int64_t)*n_dev);
    KeyRange kr{0u, 0};
    if constexpr (RANGE) kr = key_range(range, range_parts, RB);
    const unsigned nt = active_tiles<ITEMS>(n, nullptr);
    __shared__ uint32_t cnt[kWaves][R];
    const int t = threadIdx.x, wave = t >> 6;
    for (TileWalk it = tile_walk(nt); it.t < it.end; it.t += it.step) {
        const unsigned tile = it.t;
        // the tile's keys are loaded before the counters are cleared, so that their latency overlaps
        // the barriers
        const int64_t base = (int64_t)tile * (kSortBlock * ITEMS);
        K key[ITEMS];
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const int64_t idx = base + (int64_t)k * kSortBlock + t;
            key[k] = idx < n ? keys[idx] : K{};
        }
        __syncthreads();  // the previous tile's sums are read
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int j = 0; j < DPT; ++j) cnt[w][j * kSortBlock + t] = 0;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const int64_t idx = base + (int64_t)k * kSortBlock + t;
            if (idx < n) atomicAdd(&cnt[wave][pass_digit<K, RANGE>(key[k], shift, bits, kr)], 1u);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int d = j * kSortBlock + t;
            uint32_t s = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) s += cnt[w][d];
            hist[(int64_t)d * nb + tile] = s;
        }
    }
}

// one block per digit: exclusive scan of hist[d * nb .. d * nb + nt) over the nt tiles holding keys,
// total into digit_total[d]. Chunks of kSortBlock counts are scanned in order; a window of kScanWindow
// chunks is loaded before any of it is scanned (one memory round trip per window, not per chunk).
constexpr int kScanWindow = 8;
template <int ITEMS>
__global__ __launch_bounds__(kSortBlock) void radix_scan_hist(uint32_t* __restrict__ hist, unsigned nb,
                                                              uint32_t* __restrict__ digit_total, int64_t n,
                                                              const uint32_t* __restrict__ n_dev) {
    __shared__ uint32_t lds[kWaves];
    const unsigned nt = active_tiles<ITEMS>(n, n_dev);
    uint32_t* h = hist + (int64_t)blockIdx.x * nb;
    uint32_t carry = 0;
    for (unsigned w0 = 0; w0 < nt; w0 += kSortBlock * kScanWindow) {
        uint32_t v[kScanWindow];
#pragma unroll
        for (int j = 0; j < kScanWindow; ++j) {
            const unsigned i = w0 + (unsigned)(kSortBlock * j) + threadIdx.x;
            v[j] = i < nt ? h[i] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kScanWindow; ++j) {
            const unsigned start = w0 + (unsigned)(kSortBlock * j);
            if (start >= nt) break;  // block-uniform
            const unsigned i = start + threadIdx.x;
            uint32_t tot;
            const uint32_t ex = block_exclusive_scan<uint32_t>(v[j], lds, tot);
            if (i < nt) h[i] = carry + ex;
            carry += tot;
        }
    }
    if (threadIdx.x == 0) digit_total[blockIdx.x] = carry;
}

// Output policies for the downsweep scatter.
template <typename K, typename V>
struct PlainOut {
    K* keys;
    V* vals;
    XSG_DEV void put(int64_t pos, K k, V v) const { keys[pos] = k; vals[pos] = v; }
};

// Downsweep of one pass. Each wavefront ranks its own contiguous segment (ITEMS * 64 keys) of the
// block's tile in ITEMS steps of 64 keys: equal digits inside a step are found with 64-bit ballots over the
// digit bits, and a wave-private counter per digit (in LDS, no block barrier) carries the rank
// across steps. The block then combines the four waves' counts, reorders its keys by digit in
// LDS and writes them out so that consecutive lanes store consecutive addresses of a digit's run.
// Segments, steps and lanes are visited in input order, so the pass is stable.
template <typename K, typename V, typename Out, int ITEMS = kSortItems, int RB = 8, bool RANGE = false>
__global__ __launch_bounds__(kSortBlock) void radix_downsweep(const K* __restrict__ keys_in,
                                                              const V* __restrict__ vals_in, int64_t n,
                                                              int shift, int bits,
                                                              const uint32_t* __restrict__ hist,
                                                              const uint32_t* __restrict__ digit_total,
                                                              unsigned nb, Out out,
                                                              const uint32_t* __restrict__ n_dev,
                                                              const uint32_t* __restrict__ range = nullptr,
                                                              int range_parts = 0) {
    if (n_dev) n = min(n, (int64_t)*n_dev);
    KeyRange kr{0u, 0};
    if constexpr (RANGE) kr = key_range(range, range_parts, RB);
    constexpr int R = 1 << RB, DPT = R / kSortBlock;  // thread t owns digits t * DPT .. t * DPT + DPT - 1
    constexpr int kTile = kSortBlock * ITEMS;
    constexpr int kSeg = kTile / kWaves;  // keys per wave
    constexpr int kSteps = kSeg / 64;
    __shared__ uint32_t wcnt[kWaves][R];
    __shared__ uint32_t gbase[R];
    __shared__ uint32_t lpre[R];
    __shared__ uint32_t scan_lds[kWaves];
    __shared__ K skeys[kTile];
    __shared__ V svals[kTile];
    const int t = threadIdx.x, wave = t >> 6, lane = __lane_id();
    const unsigned nt = active_tiles<ITEMS>(n, nullptr);
    const int seg0 = wave * kSeg;
    // A tile's keys, values and histogram words are loaded into registers before the barriers and
    // scans that precede their use (the first tile's before the digit prefix scan, each next one's
    // while the current tile is written out), so their latency overlaps that work.
    K key[kSteps];
    V val[kSteps];
    uint32_t hcol[DPT];
    auto load_tile = [&](unsigned tile) {
        const int64_t tile0 = (int64_t)tile * kTile;
        const int n_tile = (int)min<int64_t>(kTile, n - tile0);
#pragma unroll
        for (int r = 0; r < kSteps; ++r) {
            const int li = seg0 + r * 64 + lane;
            key[r] = K{};
            val[r] = V{};
            if (li < n_tile) {
                key[r] = keys_in[tile0 + li];
                val[r] = vals_in[tile0 + li];
            }
        }
#pragma unroll
        for (int j = 0; j < DPT; ++j) hcol[j] = hist[(int64_t)(t * DPT + j) * nb + tile];
    };
    TileWalk it = tile_walk(nt);
    if (it.t < it.end) load_tile(it.t);
    uint32_t dprefix[DPT];  // first output position of each of the thread's digits
    {
        uint32_t loc[DPT], s = 0;
#pragma unroll
        for (int j = 0; j < DPT; ++j) { loc[j] = s; s += digit_total[t * DPT + j]; }
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan<uint32_t>(s, scan_lds, tot);
#pragma unroll
        for (int j = 0; j < DPT; ++j) dprefix[j] = ex + loc[j];
    }
    for (; it.t < it.end; it.t += it.step) {
        const unsigned tile = it.t;
        __syncthreads();  // the previous tile's LDS contents are consumed
        const int64_t tile0 = (int64_t)tile * kTile;
        const int n_tile = (int)min<int64_t>(kTile, n - tile0);
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int d = t * DPT + j;
            gbase[d] = dprefix[j] + hcol[j];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) wcnt[w][d] = 0;
        }
        __syncthreads();
        const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        uint32_t rank[kSteps];
#pragma unroll
        for (int r = 0; r < kSteps; ++r) {
            const int li = seg0 + r * 64 + lane;
            const bool valid = li < n_tile;
            uint32_t d = 0;
            if (valid) d = pass_digit<K, RANGE>(key[r], shift, bits, kr);
            uint64_t peers = __ballot(valid);
            for (int b = 0; b < bits; ++b) {
                const uint64_t m = __ballot((d >> b) & 1u);
                peers &= ((d >> b) & 1u) ? m : ~m;
            }
            const uint32_t before = (uint32_t)__popcll(peers & lt_mask);
            const uint32_t base = valid ? wcnt[wave][d] : 0u;
            rank[r] = base + before;
            if (valid && before == 0) wcnt[wave][d] = base + (uint32_t)__popcll(peers);
        }
        __syncthreads();
        {  // per digit: exclusive prefix over the waves, block-local exclusive prefix over digits
            uint32_t loc[DPT], s = 0;
#pragma unroll
            for (int j = 0; j < DPT; ++j) {
                const int d = t * DPT + j;
                uint32_t sd = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) { const uint32_t c = wcnt[w][d]; wcnt[w][d] = sd; sd += c; }
                loc[j] = s;
                s += sd;
            }
            uint32_t tot;
            const uint32_t ex = block_exclusive_scan<uint32_t>(s, scan_lds, tot);
#pragma unroll
            for (int j = 0; j < DPT; ++j) lpre[t * DPT + j] = ex + loc[j];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kSteps; ++r) {
            const int li = seg0 + r * 64 + lane;
            if (li < n_tile) {
                const uint32_t d = pass_digit<K, RANGE>(key[r], shift, bits, kr);
                const uint32_t pos = lpre[d] + wcnt[wave][d] + rank[r];
                skeys[pos] = key[r];
                svals[pos] = val[r];
            }
        }
        if (it.t + it.step < it.end) load_tile(it.t + it.step);  // block-uniform
        __syncthreads();
        for (int i = t; i < n_tile; i += kSortBlock) {
            const K k = skeys[i];
            const uint32_t d = pass_digit<K, RANGE>(k, shift, bits, kr);
            out.put((int64_t)gbase[d] + (i - lpre[d]), k, svals[i]);
        }
    }
}

// Runs every pass of a stable LSD sort over bits [begin_bit, end_bit) (RB-bit digits, last one
// narrower) ping-ponging between (k0, v0) and (k1, v1); the last pass goes through `final_out`.
// Returns the number of passes. hist must hold (1 << RB) * sort_blocks<ITEMS>(n) words, dtot
// 1 << RB words. With n_dev, the device-side count (at most n) is sorted; n only bounds it, so a sort whose
// count is usually far below n uses fewer ITEMS per block to spread over more blocks, and its
// grids are capped at kDevCountGrid workgroups that loop over the tiles holding keys (dispatching
// workgroups for empty tiles costs about as much as sorting a full one). With first_hist_ready, the
// caller has already stored the first pass's per-tile histograms in hist (the kernel that wrote the
// keys counted them), and the first upsweep is skipped.
constexpr unsigned kDevCountGrid = 256;
template <typename K, typename V, typename FinalOut, int ITEMS = kSortItems, int RB = 8>
inline int radix_sort_passes(K* k0, V* v0, K* k1, V* v1, int64_t n, int begin_bit, int end_bit,
                             uint32_t* hist, uint32_t* dtot, FinalOut final_out, hipStream_t s,
                             const uint32_t* n_dev = nullptr, bool first_hist_ready = false,
                             unsigned dev_grid = kDevCountGrid) {
    const unsigned nb = sort_blocks<ITEMS>(n);
    const unsigned grid = n_dev ? min(nb, dev_grid) : nb;
    int passes = 0;
    K* src_k = k0; V* src_v = v0; K* dst_k = k1; V* dst_v = v1;
    for (int shift = begin_bit; shift < end_bit; shift += RB) {
        const int bits = min(RB, end_bit - shift);
        const bool last = shift + RB >= end_bit;
        if (!(first_hist_ready && shift == begin_bit))
            radix_upsweep<K, ITEMS, RB><<<grid, kSortBlock, 0, s>>>(src_k, n, shift, bits, hist, nb, n_dev);
        radix_scan_hist<ITEMS><<<1u << RB, kSortBlock, 0, s>>>(hist, nb, dtot, n, n_dev);
        if (last) {
            radix_downsweep<K, V, FinalOut, ITEMS, RB><<<grid, kSortBlock, 0, s>>>(src_k, src_v, n, shift, bits,
                                                                                   hist, dtot, nb, final_out, n_dev);
        } else {
            radix_downsweep<K, V, PlainOut<K, V>, ITEMS, RB><<<grid, kSortBlock, 0, s>>>(
                src_k, src_v, n, shift, bits, hist, dtot, nb, PlainOut<K, V>{dst_k, dst_v}, n_dev);
        }
        ++passes;
        K* tk = src_k; src_k = dst_k; dst_k = tk;
        V* tv = src_v; src_v = dst_v; dst_v = tv;
    }
    return passes;
}

}  // namespace xsg
