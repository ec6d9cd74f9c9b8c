// Instantiation and dispatch of the prefill kernels (prefill_kernels.h).
#include "prefill_kernels.h"

#include <algorithm>

namespace llmp {
namespace {

constexpr int kAppendThreads = 256;
// Tile-image threads: the tile's K and V^T work must divide evenly (head_dim 96: 192 threads).
template <int D>
constexpr int tile_threads() { return D == 96 ? 192 : 256; }

// Launch shape of the attention kernel: one query head per wave (HPW 1, measured best at the
// C5 shape: each wave's K/V fragments feed its MFMAs while occupancy stays at 4 waves/SIMD),
// 16*NB query tokens per workgroup, at most 8 waves.  NB_BIG is used when the grid then still
// holds two workgroups per CU, else NB_BIG/2 (short prompts).
constexpr int nb_big(int G) { return G >= 8 ? 1 : (8 / G >= 4 ? 4 : 8 / G); }

// Workgroups per key split: query blocks of 16*NB tokens times KV heads.
inline int prefill_items(int P, int Hkv, int NB) { return ((P + 16 * NB - 1) / (16 * NB)) * Hkv; }

// Query blocks per workgroup the launch uses for P tokens and group size G (see launch_attn_dg).
inline int prefill_nb(int P, int Hkv, int G, int n_cu) {
    const int nb = nb_big(G);
    return (nb > 1 && prefill_items(P, Hkv, nb) < 2 * n_cu) ? nb / 2 : nb;
}

template <int D, int G, int NB>
hipError_t launch_attn_dgn(const pk::PrefillArgs& a, const uint4* ws, int tile0, int n_tiles,
                           int ksplit, int n_cu, hipStream_t stream) {
    const int items = ((a.P + 16 * NB - 1) / (16 * NB)) * a.Hkv * a.kv_rep;
    if constexpr (D == 96) {   // fp32 caches only at head_dim 96
        if (a.kq != nullptr) return hipErrorInvalidValue;
    } else if (ksplit > 1 && a.kq != nullptr) {   // few query blocks: stage from the cache
        hipLaunchKernelGGL((pk::prefill_attn2_kernel<D, G, NB, 1, true, true>), dim3(items, ksplit),
                           dim3(G * NB * 64), 0, stream, a, ws, tile0, n_tiles, ksplit);
        return hipGetLastError();
    }
    if (ksplit > 1)
        hipLaunchKernelGGL((pk::prefill_attn2_kernel<D, G, NB, 1, true>), dim3(items, ksplit),
                           dim3(G * NB * 64), 0, stream, a, ws, tile0, n_tiles, ksplit);
    else if (D == 64 && items <= n_cu)
        // At most one workgroup per CU: two key halves per workgroup (four 64-key buffers fit
        // at head_dim 64) double the waves on each CU and halve the heaviest block's chain.
        // With more query blocks than CUs two workgroups share a CU and the plain kernel is
        // faster (C5 P = 2048: 84 against 88 us; P = 512: 25.8 against 23.9 us with halves).
        hipLaunchKernelGGL((pk::prefill_attn2_kernel<D, G, NB, 1, false, false, D == 64 ? 2 : 1>),
                           dim3(items, ksplit), dim3((D == 64 ? 2 : 1) * G * NB * 64), 0, stream,
                           a, ws, tile0, n_tiles, ksplit);
    else
        hipLaunchKernelGGL((pk::prefill_attn2_kernel<D, G, NB, 1, false>), dim3(items, ksplit),
                           dim3(G * NB * 64), 0, stream, a, ws, tile0, n_tiles, ksplit);
    return hipGetLastError();
}

template <int D, int G>
hipError_t launch_attn_dg(const pk::PrefillArgs& a, const uint4* ws, int tile0, int n_tiles,
                          int n_cu, int ksplit, hipStream_t stream) {
    constexpr int NB = nb_big(G);
    if constexpr (NB > 1) {
        if (prefill_items(a.P, a.Hkv * a.kv_rep, NB) < 2 * n_cu)
            return launch_attn_dgn<D, G, NB / 2>(a, ws, tile0, n_tiles, ksplit, n_cu, stream);
    }
    return launch_attn_dgn<D, G, NB>(a, ws, tile0, n_tiles, ksplit, n_cu, stream);
}

template <int D>
hipError_t launch_attn_d(const pk::PrefillArgs& a, int group, const uint4* ws, int tile0,
                         int n_tiles, int n_cu, int ksplit, hipStream_t stream) {
    switch (group) {
    case 1: return launch_attn_dg<D, 1>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
    case 2: return launch_attn_dg<D, 2>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
    case 3: return launch_attn_dg<D, 3>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
    case 4: return launch_attn_dg<D, 4>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
    default: break;
    }
    if constexpr (D == 96) {   // decode's head_dim-96 groups: 1-4
        return hipErrorInvalidValue;
    } else {
        switch (group) {
        case 5: return launch_attn_dg<D, 5>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
        case 6: return launch_attn_dg<D, 6>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
        case 7: return launch_attn_dg<D, 7>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
        case 8: return launch_attn_dg<D, 8>(a, ws, tile0, n_tiles, n_cu, ksplit, stream);
        default: return hipErrorInvalidValue;
        }
    }
}

template <int D>
hipError_t launch_combine_d(const pk::PrefillArgs& a, int ksplit, hipStream_t stream) {
    hipLaunchKernelGGL((pk::prefill_combine_kernel<D>), dim3((unsigned)(a.P * a.Hq)),
                       dim3(pk::kCombineThreads), 0, stream, a, ksplit);
    return hipGetLastError();
}

template <int D>
hipError_t launch_tiles_d(const pk::PrefillArgs& a, uint4* ws, int tile0, int n_tiles,
                          int row_end, hipStream_t stream) {
    constexpr int NT = tile_threads<D>();
    if constexpr (D == 96) {   // fp32 caches only at head_dim 96
        if (a.kq != nullptr) return hipErrorInvalidValue;
    } else if (a.kq != nullptr) {
        hipLaunchKernelGGL((pk::prefill_tile_kernel<D, NT, true>), dim3(n_tiles, a.Hkv), dim3(NT), 0,
                           stream, a, ws, tile0, n_tiles, row_end);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((pk::prefill_tile_kernel<D, NT, false>), dim3(n_tiles, a.Hkv), dim3(NT), 0,
                       stream, a, ws, tile0, n_tiles, row_end);
    return hipGetLastError();
}

template <int D>
hipError_t launch_append_d(const pk::PrefillArgs& a, hipStream_t stream) {
    const size_t lds = pk::prefill_append_lds(a.Hkv, D);
    hipLaunchKernelGGL((pk::prefill_append_kernel<D, kAppendThreads>), dim3(a.P),
                       dim3(kAppendThreads), lds, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_append(const pk::PrefillArgs& a, int head_dim, hipStream_t stream) {
    switch (head_dim) {
    case 64: return launch_append_d<64>(a, stream);
    case 96: return launch_append_d<96>(a, stream);
    case 128: return launch_append_d<128>(a, stream);
    case 256: return launch_append_d<256>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

int prefill_tile_keys(int head_dim) {
    switch (head_dim) {
    case 64: return pk::TileLds<64>::TK;
    case 96: return pk::TileLds<96>::TK;
    case 128: return pk::TileLds<128>::TK;
    case 256: return pk::TileLds<256>::TK;
    default: return 0;
    }
}

size_t prefill_tile_bytes(int head_dim) {
    switch (head_dim) {
    case 64: return sizeof(pk::TileLds<64>);
    case 96: return sizeof(pk::TileLds<96>);
    case 128: return sizeof(pk::TileLds<128>);
    case 256: return sizeof(pk::TileLds<256>);
    default: return 0;
    }
}

hipError_t launch_prefill_tiles(const pk::PrefillArgs& a, int head_dim, void* ws, int tile0,
                                int n_tiles, int row_end, hipStream_t stream) {
    uint4* w = static_cast<uint4*>(ws);
    switch (head_dim) {
    case 64: return launch_tiles_d<64>(a, w, tile0, n_tiles, row_end, stream);
    case 96: return launch_tiles_d<96>(a, w, tile0, n_tiles, row_end, stream);
    case 128: return launch_tiles_d<128>(a, w, tile0, n_tiles, row_end, stream);
    case 256: return launch_tiles_d<256>(a, w, tile0, n_tiles, row_end, stream);
    default: return hipErrorInvalidValue;
    }
}

int prefill_key_splits(int P, int pos0, int window, int n_kv_heads, int group, int head_dim,
                       int n_cu) {
    const int TK = prefill_tile_keys(head_dim);
    if (TK <= 0 || group <= 0) return 1;
    const int items = prefill_items(P, n_kv_heads, prefill_nb(P, n_kv_heads, group, n_cu));
    if (items >= n_cu) return 1;
    // Key tiles of the last query (the heaviest workgroup's range, up to one block's spread).
    const int last = pos0 + P - 1;
    const int kbeg = window > 0 ? std::max(0, last - window + 1) : 0;
    const int tiles = last / TK - kbeg / TK + 1;
    int ks = (2 * n_cu + items - 1) / items;          // about two workgroups per CU
    ks = std::min(ks, std::max(1, tiles / 2));        // at least two tiles per split
    return std::max(1, std::min(ks, kMaxPrefillSplits));
}

hipError_t launch_prefill_attn(const pk::PrefillArgs& a, int head_dim, int group, const void* ws,
                               int tile0, int n_tiles, int n_cu, int ksplit, hipStream_t stream) {
    const uint4* w = static_cast<const uint4*>(ws);
    hipError_t e;
    switch (head_dim) {
    case 64: e = launch_attn_d<64>(a, group, w, tile0, n_tiles, n_cu, ksplit, stream); break;
    case 96: e = launch_attn_d<96>(a, group, w, tile0, n_tiles, n_cu, ksplit, stream); break;
    case 128: e = launch_attn_d<128>(a, group, w, tile0, n_tiles, n_cu, ksplit, stream); break;
    case 256: e = launch_attn_d<256>(a, group, w, tile0, n_tiles, n_cu, ksplit, stream); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || ksplit <= 1) return e;
    switch (head_dim) {
    case 64: return launch_combine_d<64>(a, ksplit, stream);
    case 96: return launch_combine_d<96>(a, ksplit, stream);
    case 128: return launch_combine_d<128>(a, ksplit, stream);
    default: return launch_combine_d<256>(a, ksplit, stream);
    }
}

}  // namespace llmp
