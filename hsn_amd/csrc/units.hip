// The remaining ops of the reference's sparse-round ABI (kernels/include/hsn_ops.h:101-153): the
// grouped unit MLP and the CSR neighbour messages, forward and backward, for f32 / f16 / bf16
// storage with fp32 arithmetic and one rounding per output.
//
// The products run on the matrix cores: v_mfma_f32_16x16x4_f32 tiles (a 16x4 by 4x16 product per
// instruction, fp32 in and out), the operands widened from the storage dtype on load, so f16 and
// bf16 inputs multiply exactly and accumulate in fp32. Lane l of a wavefront supplies A[l % 16][l
// / 16] and B[l / 16][l % 16] and receives D[4 (l / 16) + r][l % 16] in its r-th result
// register. A workgroup is four wavefronts side by side over 64 output columns.
//
// The ABI takes no workspace, so nothing is staged between launches: the grouped MLP finds each
// unit's pairs by scanning unit_idx (a wavefront-wide ballot per 64 pairs), and its backward
// recomputes the hidden cotangent dz1 tile by tile where it is consumed. Every sum runs in a fixed
// order (no atomics), so all results are reproducible run to run whatever `deterministic` says.
// CSR entries outside [0, N) / [0, E] contribute nothing (never an out-of-bounds access); the
// graph's well-formedness is the caller's, as for the reference's GPU path.
#include <algorithm>

#include "common.cuh"

#include "../../include/hsn_ops.h"
#include "abi_util.h"

namespace hsn {
// Raise a kernel's dynamic-LDS limit to 160 KiB once per (kernel, device) (runtime.cpp).
hipError_t allow_lds_raw(const void* kernel, size_t lds);

namespace units {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr float kRsqrt2 = 0.70710678118654752f;
constexpr float kRsqrt2Pi = 0.39894228040143268f;

// The exact GELU x/2 (1 + erf(x / sqrt 2)) and its derivative Phi(x) + x phi(x)
// (kernels/include/hsn_ops.h:104-113), from the device library's erff / expf.
__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erff(x * kRsqrt2)); }
__device__ __forceinline__ float gelu_grad(float x) {
    return 0.5f * (1.0f + erff(x * kRsqrt2)) + x * expf(-0.5f * x * x) * kRsqrt2Pi;
}

// The next (up to) 16 pairs p >= cur of unit j, in order: lane i < n holds the i-th, `cur`
// advances past them. Every lane of the wavefront computes the same n and cur.
struct Chunk {
    int n;
    int row;  // lane's pair (lane < n), else -1
};
__device__ __forceinline__ Chunk next_pairs(const int32_t* unit_idx, int P, int j, int& cur) {
    const int lane = lane_id();
    int n = 0, row = -1;
    while (n < 16 && cur < P) {
        const int p = cur + lane;
        uint64_t m = ballot(p < P && unit_idx[p] == j);
        int last = -1;
        while (m != 0ull && n < 16) {
            const int bit = __builtin_ctzll(m);
            m &= m - 1ull;
            if (lane == n) row = cur + bit;
            ++n;
            last = bit;
        }
        cur = m != 0ull ? cur + last + 1 : cur + 64;  // stopped early: resume after the last taken
    }
    return Chunk{n, row};
}

// The pair of A-row `i` of the chunk (or -1). A cross-lane read: call it with every lane active
// (a lane outside the exec mask does not supply its value).
__device__ __forceinline__ int pair_of(const Chunk& c, int i) { return __shfl(c.row, i, kWave); }

// dz1 = (grad_out W2[j]^T) * gelu'(z1) for the chunk's pairs and hidden columns [h0, h0 + 64)
// (each wavefront its 16), into LDS dz[16][64]; with `act`, gelu(z1) too. Rows past the chunk and
// columns past H hold zeros.
template <typename T>
__device__ __forceinline__ void dz_tile(const T* grad_out, const T* W2j, const T* hidden,
                                        const Chunk& c, int h0, int d, int H, float (*dz)[64],
                                        float (*act)[64]) {
    const int lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15, lq = lane >> 4;
    const int h = h0 + 16 * w + lr;
    const bool hin = h < H;
    const int pa = pair_of(c, lr);
    const T* go = grad_out + int64_t(pa < 0 ? 0 : pa) * d;
    const T* w2 = W2j + int64_t(hin ? h : 0) * d;  // W2[j][h][:]: B[k][h] = W2[j][h][k]
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int U = 4;
    for (int k0 = 0; k0 < d; k0 += 4 * U) {
        float a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + 4 * u + lq;
            const int kc = k < d ? k : d - 1;
            a[u] = pa >= 0 && k < d ? load_f32(go, kc) : 0.0f;
            b[u] = hin && k < d ? load_f32(w2, kc) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc = mfma(a[u], b[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * lq + r;
        const int p = pair_of(c, row);
        const float z = p >= 0 && hin ? load_f32(hidden, int64_t(p) * H + h) : 0.0f;
        const bool ok = p >= 0 && hin;
        dz[row][16 * w + lr] = ok ? acc[r] * gelu_grad(z) : 0.0f;
        if (act) act[row][16 * w + lr] = ok ? gelu(z) : 0.0f;
    }
}

// ------------------------------------------------------------------------------------------
// grouped_unit_mlp forward: (M, S) workgroups, unit j's chunks s, s + S, ... of 16 pairs
// ------------------------------------------------------------------------------------------

// For a chunk: per hidden tile of 64 columns, z1 = v W1[j] + b1[j] (saved pre-GELU, rounded once
// to the storage dtype), gelu(z1) in fp32 into LDS, and out += gelu(z1) W2[j][tile] accumulated
// in registers over the tiles; out = that + b2[j]. Layer 2 reads the fp32 activation, not the
// rounded copy, as the reference's two kernels do through an fp32 buffer.
template <typename T>
__global__ __launch_bounds__(256) void mlp_fwd(const T* v, const int32_t* unit_idx, const T* W1,
                                               const T* b1, const T* W2, const T* b2, T* hidden,
                                               T* out, int P, int d, int H) {
    __shared__ float act[16][64];
    const int j = blockIdx.x, s = blockIdx.y, S = gridDim.y;
    const int lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15, lq = lane >> 4;
    const int in = 4 * d;
    const T* W1j = W1 + int64_t(j) * in * H;
    const T* W2j = W2 + int64_t(j) * H * d;
    int cur = 0, chunk = 0;
    for (;;) {
        const Chunk c = next_pairs(unit_idx, P, j, cur);
        if (c.n == 0) break;
        if (chunk++ % S != s) continue;
        const int pa = pair_of(c, lr);
        const T* vr = v + int64_t(pa < 0 ? 0 : pa) * in;
        v4f oacc[4];  // out columns 16 (w + 4 t) + lr, t < 4 (d <= 256)
#pragma unroll
        for (int t = 0; t < 4; ++t) oacc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        for (int h0 = 0; h0 < H; h0 += 64) {
            const int hc = h0 + 16 * w + lr;
            const bool hin = hc < H;
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
            constexpr int U = 8;
            for (int k0 = 0; k0 < in; k0 += 4 * U) {
                float a[U], b[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int k = k0 + 4 * u + lq;
                    const int kc = k < in ? k : in - 1;
                    a[u] = pa >= 0 && k < in ? load_f32(vr, kc) : 0.0f;
                    b[u] = hin && k < in ? load_f32(W1j, int64_t(kc) * H + hc) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) acc = mfma(a[u], b[u], acc);
            }
            const float bias = hin ? load_f32(b1, int64_t(j) * H + hc) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * lq + r;
                const int p = pair_of(c, row);
                const float z = acc[r] + bias;
                const bool ok = p >= 0 && hin;
                if (ok) store_f32(hidden, int64_t(p) * H + hc, z);
                act[row][16 * w + lr] = ok ? gelu(z) : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int oc = 16 * (w + 4 * t) + lr;
                if (16 * (w + 4 * t) < d) {  // uniform in the wavefront
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const int k = 4 * q + lq;
                        const float av = act[lr][k];
                        const float bv = h0 + k < H && oc < d ? load_f32(W2j, int64_t(h0 + k) * d + oc) : 0.0f;
                        oacc[t] = mfma(av, bv, oacc[t]);
                    }
                }
            }
            __syncthreads();
        }
        int prow[4];  // the output rows' pairs (a cross-lane read: every lane takes part)
#pragma unroll
        for (int r = 0; r < 4; ++r) prow[r] = pair_of(c, 4 * lq + r);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int oc = 16 * (w + 4 * t) + lr;
            if (oc < d) {
                const float bias = load_f32(b2, int64_t(j) * d + oc);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (prow[r] >= 0) store_f32(out, int64_t(prow[r]) * d + oc, oacc[t][r] + bias);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// grouped_unit_mlp forward by row tiles (d a multiple of 4, P <= 16384, M <= 4096)
// ------------------------------------------------------------------------------------------

// The row tiles of every unit's pairs (16 pairs of one unit in pair order, laid end to end unit
// after unit; a workgroup finds its tile from LDS counts of each unit's pairs), one workgroup each,
// all H hidden columns walked in tiles of 64. The first layer's reduction over the 4d inputs is
// split over the four wavefronts (each lane group g a contiguous quarter of a wavefront's share);
// a lane's 16-byte load of W1[j][k][h0 + 4 lr ..] feeds four interleaved column tiles (tile t's
// column lr is h0 + 4 lr + t), and the next 16 steps' weights are in flight while a block's
// products run, across the hidden tiles too. The shares are summed in wavefront order, z1 stored
// (rounded once), gelu(z1) kept in fp32 in LDS, and out += gelu(z1) W2[j][tile] accumulated in
// registers over the tiles, a 16-column output tile a wavefront.
constexpr int kTileMaxSlots = 16384;
constexpr int kTileMaxUnits = 4096;
constexpr int kTileBlock = 8;  // reduction steps whose weights are loaded together

struct TileLds {
    int ucache, count, rows, meta, vs, red, act, b1, sv, bytes;
};
__host__ __device__ inline TileLds tile_lds(int P, int M, int d, int H) {
    TileLds L;
    L.sv = 4 * d + 1;
    L.ucache = 0;                                         // uint16 [P]: each pair's unit
    L.count = (2 * P + 15) / 16 * 16;                     // int [M]
    L.rows = L.count + (4 * M + 15) / 16 * 16;            // int [16]
    L.meta = L.rows + 64;                                 // int [4]
    L.vs = L.meta + 16;                                   // float [16][sv]
    L.red = L.vs + 4 * 16 * L.sv;                         // float [4][16][65]
    L.act = L.red + 4 * 4 * 16 * 65;                      // float [16][65]
    L.b1 = L.act + 4 * 16 * 65;                           // float [H]: the unit's first-layer bias
    L.bytes = L.b1 + 4 * H;
    return L;
}

// Four consecutive values of a row from column c on, widened; 0 past `cols`.
template <typename T>
__device__ __forceinline__ float4 row4w(const T* w, int c, int cols, bool aligned) {
    if (aligned && c + 4 <= cols) {
        if constexpr (sizeof(T) == 4) {
            return *reinterpret_cast<const float4*>(w + c);
        } else {
            const uint2 raw = *reinterpret_cast<const uint2*>(w + c);
            T e[4];
            __builtin_memcpy(e, &raw, 8);
            return make_float4(to_f32(e[0]), to_f32(e[1]), to_f32(e[2]), to_f32(e[3]));
        }
    }
    return make_float4(c < cols ? to_f32(w[c]) : 0.0f, c + 1 < cols ? to_f32(w[c + 1]) : 0.0f,
                       c + 2 < cols ? to_f32(w[c + 2]) : 0.0f,
                       c + 3 < cols ? to_f32(w[c + 3]) : 0.0f);
}

// The workgroup's row tile (blockIdx.x over every unit's tiles of 16 pairs, laid end to end unit
// after unit): returns its unit, or -1 past the last tile, with its pairs in rows[16] (-1 past
// the unit's pairs), from LDS counts of each unit's pairs. Every thread of the workgroup calls it.
__device__ __forceinline__ int find_row_tile(const int32_t* unit_idx, int P, int M,
                                             uint16_t* ucache, int* count, int* rows, int* meta) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int j = tid; j < M; j += 256) count[j] = 0;
    for (int q = tid; q < P; q += 256) {
        const int u = unit_idx[q];
        ucache[q] = u >= 0 && u < M ? static_cast<uint16_t>(u) : uint16_t(0xffff);
    }
    __syncthreads();
    for (int q = tid; q < P; q += 256)  // integer counts: any order gives the same
        if (ucache[q] != 0xffff) atomicAdd(&count[ucache[q]], 1);
    __syncthreads();
    if (wave == 0) {
        int unit = -1, tile = 0;
        if (lane == 0) {
            int before = 0;
            for (int j = 0; j < M; ++j) {
                const int t = (count[j] + 15) / 16;
                if (static_cast<int>(blockIdx.x) < before + t) {
                    unit = j;
                    tile = blockIdx.x - before;
                    break;
                }
                before += t;
            }
        }
        unit = __builtin_amdgcn_readfirstlane(unit);
        tile = __builtin_amdgcn_readfirstlane(tile);
        if (lane < 16) rows[lane] = -1;
        if (unit >= 0) {
            const int first = tile * 16;
            int base = 0;
            for (int q0 = 0; q0 < P && base < first + 16; q0 += kWave) {
                const int q = q0 + lane;
                const bool mine = q < P && ucache[q] == unit;
                const uint64_t m = ballot(mine);
                const int rank = base + lanes_below(m);
                if (mine && rank >= first && rank < first + 16) rows[rank - first] = q;
                base += __popcll(m);
            }
        }
        if (lane == 0) meta[0] = unit;
    }
    __syncthreads();
    return meta[0];
}

template <typename T, bool ALIGNED, bool SPLIT = false>  // ALIGNED: H % 4 == 0, rows of W1 in
// 16-byte pieces; SPLIT: one hidden tile a workgroup (blockIdx.y), z1 stored, no second layer
__global__ __launch_bounds__(256) void mlp_fwd_tiles(const T* v, const int32_t* unit_idx,
                                                     const T* W1, const T* b1, const T* W2,
                                                     const T* b2, T* hidden, T* out, int P, int M,
                                                     int d, int H) {
    extern __shared__ __align__(16) unsigned char lds[];
    const TileLds L = tile_lds(P, M, d, H);
    uint16_t* ucache = reinterpret_cast<uint16_t*>(lds + L.ucache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* vs = reinterpret_cast<float*>(lds + L.vs);
    float* red = reinterpret_cast<float*>(lds + L.red);
    float* act = reinterpret_cast<float*>(lds + L.act);
    float* b1c = reinterpret_cast<float*>(lds + L.b1);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, g = lane >> 4;
    const int n = 4 * d;

    const int j = find_row_tile(unit_idx, P, M, ucache, count, rows, meta);
    if (j < 0) return;  // past the last tile (uniform)

    // ---- the tile's inputs, widened into LDS ----
    {
        const int n4 = n / 4;
        const bool valign = (reinterpret_cast<uintptr_t>(v) & (4 * sizeof(T) - 1)) == 0;
#pragma unroll 4
        for (int e = tid; e < 16 * n4; e += 256) {
            const int pp = e / n4, c = 4 * (e % n4);
            const int q = rows[pp];
            const float4 t = q >= 0 ? row4w(v + int64_t(q) * n, c, n, valign)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float* dst = vs + pp * L.sv + c;
            dst[0] = t.x, dst[1] = t.y, dst[2] = t.z, dst[3] = t.w;
        }
    }

    const int q1 = n / 16;                       // a lane group's steps of its wavefront's share
    const int k1 = wave * (n / 4) + g * q1;      // their first input row
    constexpr bool al = ALIGNED;
    const T* W1j = W1 + int64_t(j) * n * H;
    const T* W2j = W2 + int64_t(j) * H * d;
    const int tiles_h = (H + 63) / 64;
    const int blocks = (q1 + kTileBlock - 1) / kTileBlock;  // per hidden tile
    const int tiles_d = (d + 15) / 16;
    v4f oacc[4];  // output column tiles wave, wave + 4, ... (d <= 256)
#pragma unroll
    for (int t = 0; t < 4; ++t) oacc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    auto load_block = [&](float4 (&b)[kTileBlock], int ht, int bi) {
        const int c = ht * 64 + 4 * lr;
#pragma unroll
        for (int i = 0; i < kTileBlock; ++i) {
            const int s = bi * kTileBlock + i;
            b[i] = s < q1 ? row4w(W1j + int64_t(k1 + s) * H, c, H, al)
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    // The first layer's weights stream as one sequence of blocks (`blocks` a hidden tile, tile
    // after tile); block i + 1 is loaded while block i's products run, into the other of two
    // buffers (no copy, so no wait on loads in flight), and a tile's last block is followed by
    // its tail: the shares' sum, z1, the GELU and the second layer.
    float4 bufA[kTileBlock], bufB[kTileBlock];
    load_block(bufA, SPLIT ? int(blockIdx.y) : 0, 0);
    for (int c = tid; c < H; c += 256) b1c[c] = load_f32(b1, int64_t(j) * H + c);
    __syncthreads();  // the inputs and the bias are in LDS

    v4f acc[4];
    const float* arow = vs + lr * L.sv + k1;
    const int total = SPLIT ? blocks : tiles_h * blocks;
    auto load_w2 = [&](float (&w)[16], int h0, int t) {
        const int col = (wave + 4 * t) * 16 + lr;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int h = h0 + g * 16 + s;
            w[s] = wave + 4 * t < tiles_d && col < d && h < H
                       ? load_f32(W2j, int64_t(h) * d + col) : 0.0f;
        }
    };
    auto step = [&](int i, float4 (&cur)[kTileBlock], float4 (&nxt)[kTileBlock]) {
        const int ht = SPLIT ? int(blockIdx.y) : i / blocks, bi = i % blocks;
        if (bi == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (i + 1 < total)
            load_block(nxt, SPLIT ? int(blockIdx.y) : (i + 1) / blocks, (i + 1) % blocks);
        float av[kTileBlock];
#pragma unroll
        for (int k = 0; k < kTileBlock; ++k) {
            const int s = bi * kTileBlock + k;
            av[k] = s < q1 ? arow[s] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kTileBlock; ++k) {
            acc[0] = mfma(av[k], cur[k].x, acc[0]);
            acc[1] = mfma(av[k], cur[k].y, acc[1]);
            acc[2] = mfma(av[k], cur[k].z, acc[2]);
            acc[3] = mfma(av[k], cur[k].w, acc[3]);
        }
        if (bi + 1 < blocks) return;
        // the tile's tail; its second-layer weights (the wavefront's first output tile; d <= 64:
        // all of them) are in flight during the shares' sum
        const int h0 = ht * 64;
        float w2v[16];
        if constexpr (!SPLIT) load_w2(w2v, h0, 0);
        // the wavefront's share: row 4 g + r, column 4 lr + t of the tile
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[((wave * 16) + 4 * g + r) * 65 + 4 * lr + t] = acc[t][r];
        __syncthreads();
        for (int e = tid; e < 16 * 64; e += 256) {  // the shares in wavefront order
            const int row = e >> 6, c = e & 63;
            float z = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) z += red[(w * 16 + row) * 65 + c];
            const int q = rows[row];
            if (h0 + c < H) z += b1c[h0 + c];
            const bool ok = q >= 0 && h0 + c < H;
            if (ok) store_f32(hidden, int64_t(q) * H + h0 + c, z);
            act[row * 65 + c] = ok ? gelu(z) : 0.0f;
        }
        if constexpr (SPLIT) return;
        __syncthreads();
        // out += gelu(z1) W2[j][h0 .. h0 + 63]: output tile wave + 4 t, B[k][col] = W2[j][h0 + k][col]
        {
            const float* ar = act + lr * 65 + g * 16;
            float a2[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) a2[s] = ar[s];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (wave + 4 * t < tiles_d) {  // uniform in the wavefront
                    if (t > 0) load_w2(w2v, h0, t);
#pragma unroll
                    for (int s = 0; s < 16; ++s) oacc[t] = mfma(a2[s], w2v[s], oacc[t]);
                }
            }
        }
        __syncthreads();  // red and act are rewritten by the next tile
    };
    for (int i = 0; i < total; i += 2) {
        step(i, bufA, bufB);
        if (i + 1 < total) step(i + 1, bufB, bufA);
    }
    if constexpr (SPLIT) return;
    int prow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) prow[r] = rows[4 * g + r];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int col = (wave + 4 * t) * 16 + lr;
        if (wave + 4 * t < tiles_d && col < d) {
            const float bias = load_f32(b2, int64_t(j) * d + col);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (prow[r] >= 0) store_f32(out, int64_t(prow[r]) * d + col, oacc[t][r] + bias);
        }
    }
}

// The second layer by (row tile, 16 output columns) workgroups, from the stored z1 (fp32
// storage, so z1 is exact): out = gelu(z1) W2[j] + b2[j]. The tile's gelu(z1) for all H columns
// goes into LDS; wavefront w takes hidden tiles w, w + 4, ... (their W2 columns loaded in one
// batch while the activations are staged), and the four shares are summed in wavefront order.
constexpr int kOutGroup = 4;  // hidden tiles a wavefront loads together
struct OutLds {
    int ucache, count, rows, meta, red, act, bytes;
};
__host__ __device__ inline OutLds out_lds(int P, int M, int H) {
    OutLds L;
    L.ucache = 0;                                   // uint16 [P]
    L.count = (2 * P + 15) / 16 * 16;               // int [M]
    L.rows = L.count + (4 * M + 15) / 16 * 16;      // int [16]
    L.meta = L.rows + 64;                           // int [4]
    L.red = L.meta + 16;                            // float [4][16][16]
    L.act = L.red + 4 * 4 * 16 * 16;                // float [16][H + 1]
    L.bytes = L.act + 4 * 16 * (H + 1);
    return L;
}

template <typename T>
__global__ __launch_bounds__(256) void mlp_out_tiles(const int32_t* unit_idx, const T* W2,
                                                     const T* b2, const T* hidden, T* out, int P,
                                                     int M, int d, int H) {
    extern __shared__ __align__(16) unsigned char lds[];
    const OutLds L = out_lds(P, M, H);
    uint16_t* ucache = reinterpret_cast<uint16_t*>(lds + L.ucache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* red = reinterpret_cast<float*>(lds + L.red);
    float* act = reinterpret_cast<float*>(lds + L.act);
    const int j = find_row_tile(unit_idx, P, M, ucache, count, rows, meta);
    if (j < 0) return;  // past the last tile (uniform)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, g = lane >> 4;
    const int sa = H + 1, tiles_h = (H + 63) / 64;
    const int col = blockIdx.y * 16 + lr;
    const T* W2j = W2 + int64_t(j) * H * d;
    float wv[kOutGroup][16];
    auto load_batch = [&](int base) {  // hidden tiles base + wave + 4 x (zeros past H)
#pragma unroll
        for (int x = 0; x < kOutGroup; ++x)
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int h = (base + wave + 4 * x) * 64 + g * 16 + s;
                wv[x][s] = col < d && h < H ? load_f32(W2j, int64_t(h) * d + col) : 0.0f;
            }
    };
    load_batch(0);
    {  // gelu(z1) of the tile's 16 pairs into LDS: 16 threads a row, each row's loads together
        const int row = tid >> 4, c0 = tid & 15;
        const int q = rows[row];
        const T* hr = hidden + int64_t(q < 0 ? 0 : q) * H;
        for (int cb = 0; cb < H; cb += 512) {
            float z[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int c = cb + c0 + 16 * i;
                z[i] = q >= 0 && c < H ? load_f32(hr, c) : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int c = cb + c0 + 16 * i;
                if (c < H) act[row * sa + c] = q >= 0 ? gelu(z[i]) : 0.0f;
            }
        }
    }
    __syncthreads();  // act is in LDS
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 0; base < tiles_h; base += 4 * kOutGroup) {
        if (base > 0) load_batch(base);
#pragma unroll
        for (int x = 0; x < kOutGroup; ++x) {
            const int h0 = (base + wave + 4 * x) * 64;
            if (h0 < H) {  // uniform in the wavefront
                const float* ar = act + lr * sa + h0 + g * 16;
                float av[16];
#pragma unroll
                for (int s = 0; s < 16; ++s) av[s] = h0 + g * 16 + s < H ? ar[s] : 0.0f;
#pragma unroll
                for (int s = 0; s < 16; ++s) acc = mfma(av[s], wv[x][s], acc);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 16 + 4 * g + r) * 16 + lr] = acc[r];
    __syncthreads();
    if (wave == 0 && col < d) {
        const float bias = load_f32(b2, int64_t(j) * d + col);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r, q = rows[row];
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) sum += red[(w * 16 + row) * 16 + lr];
            if (q >= 0) store_f32(out, int64_t(q) * d + col, sum + bias);
        }
    }
}

// The backward's grad_v in two launches when dz1 has fp32 room (the caller's grad_W2, written only
// afterwards): mlp_dz_tiles stores dz1 = (grad_out W2[j]^T) * gelu'(z1) for (row tile, 64 hidden
// columns) workgroups, then mlp_gv_tiles forms grad_v = dz1 W1[j]^T for (row tile, 16 inputs)
// workgroups, the hidden tiles split over the wavefronts and summed in wavefront order.
struct DzLds {
    int ucache, count, rows, meta, go, bytes;
};
__host__ __device__ inline DzLds dz_lds(int P, int M, int d) {
    DzLds L;
    L.ucache = 0;                                   // uint16 [P]
    L.count = (2 * P + 15) / 16 * 16;               // int [M]
    L.rows = L.count + (4 * M + 15) / 16 * 16;      // int [16]
    L.meta = L.rows + 64;                           // int [4]
    L.go = L.meta + 16;                             // float [16][d]: the rows' grad_out
    L.bytes = L.go + 4 * 16 * d;
    return L;
}

template <typename T>
__global__ __launch_bounds__(256) void mlp_dz_tiles(const int32_t* unit_idx, const T* W2,
                                                    const T* hidden, const T* grad_out, float* dz,
                                                    int P, int M, int d, int H) {
    extern __shared__ __align__(16) unsigned char lds[];
    const DzLds L = dz_lds(P, M, d);
    uint16_t* ucache = reinterpret_cast<uint16_t*>(lds + L.ucache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* go = reinterpret_cast<float*>(lds + L.go);
    const int j = find_row_tile(unit_idx, P, M, ucache, count, rows, meta);
    if (j < 0) return;  // past the last tile (uniform)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, g = lane >> 4;
    const int h = blockIdx.y * 64 + 16 * wave + lr;
    const bool hin = h < H;
    const T* w2h = W2 + (int64_t(j) * H + (hin ? h : 0)) * d;  // B[k][h] = W2[j][h][k]
    float b[16], z[4];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k = 4 * u + g;
        b[u] = hin && k < d ? load_f32(w2h, k) : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int q = rows[4 * g + r];
        z[r] = q >= 0 && hin ? load_f32(hidden, int64_t(q) * H + h) : 0.0f;
    }
    {  // the rows' grad_out into LDS, 16 threads a row
        const int row = tid >> 4, c0 = tid & 15, q = rows[row];
        float gr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = c0 + 16 * i;
            gr[i] = q >= 0 && c < d ? load_f32(grad_out, int64_t(q) * d + c) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (c0 + 16 * i < d) go[row * d + c0 + 16 * i] = gr[i];
    }
    __syncthreads();
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k = 4 * u + g;
        acc = mfma(k < d ? go[lr * d + k] : 0.0f, b[u], acc);
    }
    for (int k0 = 64; k0 < d; k0 += 64) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int k = k0 + 4 * u + g;
            acc = mfma(k < d ? go[lr * d + k] : 0.0f, hin && k < d ? load_f32(w2h, k) : 0.0f, acc);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int q = rows[4 * g + r];
        if (q >= 0 && hin) dz[int64_t(q) * H + h] = acc[r] * gelu_grad(z[r]);
    }
}

struct GvLds {
    int ucache, count, rows, meta, red, dz, bytes;
};
__host__ __device__ inline GvLds gv_lds(int P, int M, int H) {
    GvLds L;
    L.ucache = 0;                                   // uint16 [P]
    L.count = (2 * P + 15) / 16 * 16;               // int [M]
    L.rows = L.count + (4 * M + 15) / 16 * 16;      // int [16]
    L.meta = L.rows + 64;                           // int [4]
    L.red = L.meta + 16;                            // float [4][16][16]
    L.dz = L.red + 4 * 4 * 16 * 16;                 // float [16][H + 1]
    L.bytes = L.dz + 4 * 16 * (H + 1);
    return L;
}

template <typename T>
__global__ __launch_bounds__(256) void mlp_gv_tiles(const int32_t* unit_idx, const T* W1,
                                                    const float* dz, T* grad_v, int P, int M,
                                                    int d, int H) {
    extern __shared__ __align__(16) unsigned char lds[];
    const GvLds L = gv_lds(P, M, H);
    uint16_t* ucache = reinterpret_cast<uint16_t*>(lds + L.ucache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* red = reinterpret_cast<float*>(lds + L.red);
    float* dzs = reinterpret_cast<float*>(lds + L.dz);
    const int j = find_row_tile(unit_idx, P, M, ucache, count, rows, meta);
    if (j < 0) return;  // past the last tile (uniform)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, g = lane >> 4;
    const int n = 4 * d, sa = H + 1, tiles_h = (H + 63) / 64;
    const int i = blockIdx.y * 16 + lr;  // the input column
    const T* w1i = W1 + (int64_t(j) * n + (i < n ? i : 0)) * H;  // B[k][i] = W1[j][i][h]
    const bool al = (H % 4) == 0 && (reinterpret_cast<uintptr_t>(W1) & (4 * sizeof(T) - 1)) == 0;
    float wv[kOutGroup][16];
    auto load_batch = [&](int base) {  // hidden tiles base + wave + 4 x (zeros past H)
#pragma unroll
        for (int x = 0; x < kOutGroup; ++x)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int h = (base + wave + 4 * x) * 64 + g * 16 + 4 * q4;
                const float4 t = i < n ? row4w(w1i, h, H, al) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                wv[x][4 * q4] = t.x, wv[x][4 * q4 + 1] = t.y, wv[x][4 * q4 + 2] = t.z,
                wv[x][4 * q4 + 3] = t.w;
            }
    };
    load_batch(0);
    {  // the rows' dz1 into LDS: 16 threads a row, each row's loads together
        const int row = tid >> 4, c0 = tid & 15, q = rows[row];
        const float* zr = dz + int64_t(q < 0 ? 0 : q) * H;
        for (int cb = 0; cb < H; cb += 512) {
            float zz[32];
#pragma unroll
            for (int x = 0; x < 32; ++x) {
                const int c = cb + c0 + 16 * x;
                zz[x] = q >= 0 && c < H ? zr[c] : 0.0f;
            }
#pragma unroll
            for (int x = 0; x < 32; ++x) {
                const int c = cb + c0 + 16 * x;
                if (c < H) dzs[row * sa + c] = zz[x];
            }
        }
    }
    __syncthreads();
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 0; base < tiles_h; base += 4 * kOutGroup) {
        if (base > 0) load_batch(base);
#pragma unroll
        for (int x = 0; x < kOutGroup; ++x) {
            const int h0 = (base + wave + 4 * x) * 64;
            if (h0 < H) {  // uniform in the wavefront
                const float* ar = dzs + lr * sa + h0 + g * 16;
                float av[16];
#pragma unroll
                for (int s2 = 0; s2 < 16; ++s2) av[s2] = h0 + g * 16 + s2 < H ? ar[s2] : 0.0f;
#pragma unroll
                for (int s2 = 0; s2 < 16; ++s2) acc = mfma(av[s2], wv[x][s2], acc);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 16 + 4 * g + r) * 16 + lr] = acc[r];
    __syncthreads();
    if (wave == 0 && i < n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r, q = rows[row];
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) sum += red[(w * 16 + row) * 16 + lr];
            if (q >= 0) store_f32(grad_v, int64_t(q) * n + i, sum);
        }
    }
}

// ------------------------------------------------------------------------------------------
// grouped_unit_mlp backward
// ------------------------------------------------------------------------------------------

// (H / 64, M, 4d / 64) workgroups: unit j's hidden columns [h0, h0 + 64) and input rows
// [i0, i0 + 64): grad_W1[j][i0.., h0..] = sum_p v[p]^T dz1[p]; the first input block also
// grad_W2[j][h0.., :] = sum_p gelu(z1[p])^T grad_out[p] and grad_b1[j][h0..]; the first of all
// grad_b2[j]. A unit without pairs gets zeros.
template <typename T>
__global__ __launch_bounds__(256) void mlp_dw(const T* v, const int32_t* unit_idx, const T* W2,
                                              const T* hidden, const T* grad_out, T* grad_W1,
                                              T* grad_b1, T* grad_W2, T* grad_b2, int P, int d,
                                              int H) {
    __shared__ float dz[16][64];
    __shared__ float act[16][64];
    __shared__ float gos[16 * 256];  // the chunk's grad_out rows, [16][d]
    __shared__ float vs[16][64];     // the chunk's v rows at the workgroup's 64 inputs
    const int j = blockIdx.y, lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15,
              lq = lane >> 4, tid = threadIdx.x;
    const int in = 4 * d;
    const int h0 = blockIdx.x * 64, i0 = blockIdx.z * 64;
    const bool first_in = blockIdx.z == 0;
    const T* W2j = W2 + int64_t(j) * H * d;
    constexpr int kMaxD16 = 16;  // d <= 256: 16 column tiles of grad_W2 per wavefront
    const int nd = (d + 15) / 16;
    v4f gw1[4], gw2[kMaxD16];
#pragma unroll
    for (int t = 0; t < 4; ++t) gw1[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < kMaxD16; ++t) gw2[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float gb1 = 0.0f;  // thread tid < 64: column h0 + tid
    float gb2[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // first workgroup: columns tid + 256 u
    // each pair's unit in LDS (P <= kDwCache), so a chunk's scan reads no global memory
    constexpr int kDwCache = 16384;
    __shared__ uint16_t ucache[kDwCache];
    const bool cached = P <= kDwCache;
    if (cached) {
        for (int q0 = 0; q0 < P; q0 += 256 * 8) {
            int uu[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = q0 + tid + 256 * i;
                uu[i] = q < P ? unit_idx[q] : -1;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = q0 + tid + 256 * i;
                if (q < P)
                    ucache[q] = uu[i] >= 0 && uu[i] < 0xffff ? static_cast<uint16_t>(uu[i])
                                                             : static_cast<uint16_t>(0xffff);
            }
        }
    }
    __syncthreads();
    // the unit's next 16 pairs from `at` on, in pair order (next_pairs over the LDS copy)
    auto next = [&](int& at) -> Chunk {
        int n = 0, row = -1;
        while (n < 16 && at < P) {
            const int p = at + lane;
            const bool hit = p < P && (cached ? int(ucache[p]) == j : unit_idx[p] == j);
            uint64_t m = ballot(hit);
            int last = -1;
            while (m != 0ull && n < 16) {
                const int bit = __builtin_ctzll(m);
                m &= m - 1ull;
                if (lane == n) row = at + bit;
                ++n;
                last = bit;
            }
            at = m != 0ull ? at + last + 1 : at + 64;  // stopped early: resume after the last taken
        }
        return Chunk{n, row};
    };
    int cur = 0;
    const int hw = h0 + 16 * w + lr;  // the wavefront's hidden column for dz
    const bool hwin = hw < H;
    const T* w2h = W2j + int64_t(hwin ? hw : 0) * d;
    const int kr = tid >> 4, kc = tid & 15;  // the thread's row and column phase when staging
    float b[16];  // dz's B operand W2[j][h][k] for k < 64: the same for every chunk
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int k = 4 * u + lq;
        b[u] = hwin && k < d ? load_f32(w2h, k) : 0.0f;
    }
    // a chunk's loads in one batch: its pairs' grad_out rows and v's 64 inputs (for LDS), z1 of
    // the wavefront's rows; the next chunk's batch is issued before this chunk's products
    float gr[16], vr[4], z[4];
    auto load_chunk = [&](const Chunk& c) {
        const int pr = pair_of(c, kr);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int o = kc + 16 * i;
            gr[i] = pr >= 0 && o < d ? load_f32(grad_out, int64_t(pr) * d + o) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int x = i0 + kc + 16 * i;
            vr[i] = pr >= 0 && x < in ? load_f32(v, int64_t(pr) * in + x) : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = pair_of(c, 4 * lq + r);
            z[r] = p >= 0 && hwin ? load_f32(hidden, int64_t(p) * H + hw) : 0.0f;
        }
    };
    Chunk c = next(cur);
    if (c.n > 0) load_chunk(c);
    while (c.n > 0) {  // uniform
        const Chunk cn = next(cur);
        __syncthreads();  // the last chunk's reads of the tiles are done
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int o = kc + 16 * i;
            if (o < d) gos[kr * d + o] = gr[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) vs[kr][kc + 16 * i] = vr[i];
        float zc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) zc[r] = z[r];
        if (cn.n > 0) load_chunk(cn);  // uniform
        __syncthreads();
        // dz1 = (grad_out W2[j]^T) * gelu'(z1): A[pair][k] = grad_out rows (LDS), B[k][h] = W2
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int k = 4 * u + lq;
            acc = mfma(k < d ? gos[lr * d + k] : 0.0f, b[u], acc);
        }
        for (int k0 = 64; k0 < d; k0 += 64) {  // d above 64: the next blocks of W2's columns
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int k = k0 + 4 * u + lq;
                const float bv = hwin && k < d ? load_f32(w2h, k) : 0.0f;
                acc = mfma(k < d ? gos[lr * d + k] : 0.0f, bv, acc);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * lq + r;
            const bool ok = pair_of(c, row) >= 0 && hwin;
            dz[row][16 * w + lr] = ok ? acc[r] * gelu_grad(zc[r]) : 0.0f;
            if (first_in) act[row][16 * w + lr] = ok ? gelu(zc[r]) : 0.0f;
        }
        __syncthreads();
        // grad_W1[i][h] += sum_k v[p_k][i] dz[k][h]: A = v^T (rows i, k = pairs), B = dz
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int k = 4 * s2 + lq;  // the pair
            const float bv = dz[k][16 * w + lr];
#pragma unroll
            for (int t = 0; t < 4; ++t) gw1[t] = mfma(vs[k][16 * t + lr], bv, gw1[t]);
        }
        if (first_in) {
            // grad_W2[h][o] += sum_k gelu(z1)[k][h] grad_out[p_k][o]: A = act^T, B = grad_out
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const int k = 4 * s2 + lq;
                const float av = act[k][16 * w + lr];
#pragma unroll
                for (int t = 0; t < kMaxD16; ++t) {
                    if (t < nd) {
                        const int o = 16 * t + lr;
                        gw2[t] = mfma(av, o < d ? gos[k * d + o] : 0.0f, gw2[t]);
                    }
                }
            }
            if (tid < 64)
                for (int k = 0; k < c.n; ++k) gb1 += dz[k][tid];
            if (blockIdx.x == 0) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int o = tid + 256 * u;
                    if (o < d)
                        for (int k = 0; k < c.n; ++k) gb2[u] += gos[k * d + o];
                }
            }
        }
        c = cn;
    }
    const int h = h0 + 16 * w + lr;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i0 + 16 * t + 4 * lq + r;
            if (i < in && h < H) store_f32(grad_W1, (int64_t(j) * in + i) * H + h, gw1[t][r]);
        }
    if (first_in) {
#pragma unroll
        for (int t = 0; t < kMaxD16; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int hr = h0 + 16 * w + 4 * lq + r, o = 16 * t + lr;
                if (t < nd && hr < H && o < d)
                    store_f32(grad_W2, (int64_t(j) * H + hr) * d + o, gw2[t][r]);
            }
        if (tid < 64 && h0 + tid < H) store_f32(grad_b1, int64_t(j) * H + h0 + tid, gb1);
        if (blockIdx.x == 0)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int o = tid + 256 * u;
                if (o < d) store_f32(grad_b2, int64_t(j) * d + o, gb2[u]);
            }
    }
}

// (4d / 64, M) workgroups: grad_v[p][i0..] = sum_h dz1[p][h] W1[j][i][h], dz1 recomputed per
// hidden tile of 64.
template <typename T>
__global__ __launch_bounds__(256) void mlp_dv(const int32_t* unit_idx, const T* W1, const T* W2,
                                              const T* hidden, const T* grad_out, T* grad_v,
                                              int P, int d, int H) {
    __shared__ float dz[16][64];
    const int j = blockIdx.y, lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15,
              lq = lane >> 4;
    const int in = 4 * d;
    const int i = blockIdx.x * 64 + 16 * w + lr;
    const bool iin = i < in;
    const T* W1r = W1 + (int64_t(j) * in + (iin ? i : 0)) * H;  // W1[j][i][:]
    const T* W2j = W2 + int64_t(j) * H * d;
    int cur = 0;
    for (;;) {
        const Chunk c = next_pairs(unit_idx, P, j, cur);
        if (c.n == 0) break;
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int h0 = 0; h0 < H; h0 += 64) {
            dz_tile<T>(grad_out, W2j, hidden, c, h0, d, H, dz, nullptr);
            __syncthreads();
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int h = h0 + 4 * s + lq;
                const float av = dz[lr][4 * s + lq];
                const float bv = iin && h < H ? load_f32(W1r, h) : 0.0f;
                acc = mfma(av, bv, acc);
            }
            __syncthreads();
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = pair_of(c, 4 * lq + r);
            if (p >= 0 && iin) store_f32(grad_v, int64_t(p) * in + i, acc[r]);
        }
    }
}

// grad_v by row tiles (the forward's conditions): (row tile, 64-input group) workgroups. Per
// hidden tile of 64: dz1 = (grad_out W2[j]^T) * gelu'(z1) for the tile's 16 pairs (a 16-column
// hidden tile a wavefront, reduction over d), then grad_v[:, i0 .. i0 + 63] += dz1 W1[j]^T (a
// 16-column input tile a wavefront, reduction over the 64 hidden units). Both weight fragments
// are read along a lane's own row (16-byte loads), and the next hidden tile's fragments and z1
// values are in flight during the current tile.
struct DvLds {
    int ucache, count, rows, meta, go, dz, z, sg, bytes;
};
__host__ __device__ inline DvLds dv_lds(int P, int M, int d) {
    DvLds L;
    L.sg = d + 1;
    L.ucache = 0;                                 // uint16 [P]
    L.count = (2 * P + 15) / 16 * 16;             // int [M]
    L.rows = L.count + (4 * M + 15) / 16 * 16;    // int [16]
    L.meta = L.rows + 64;                         // int [4]
    L.go = L.meta + 16;                           // float [16][sg]: the rows' grad_out
    L.dz = L.go + 4 * 16 * L.sg;                  // float [16][65]: dz1 of a hidden tile
    L.z = L.dz + 4 * 16 * 65;                     // float [16][65]: gelu'(z1) of a hidden tile
    L.bytes = L.z + 4 * 16 * 65;
    return L;
}

template <typename T, bool ALIGNED>  // ALIGNED: rows of W1 and W2 in 16-byte pieces
__global__ __launch_bounds__(256) void mlp_dv_tiles(const int32_t* unit_idx, const T* W1,
                                                    const T* W2, const T* hidden,
                                                    const T* grad_out, T* grad_v, int P, int M,
                                                    int d, int H) {
    extern __shared__ __align__(16) unsigned char lds[];
    const DvLds L = dv_lds(P, M, d);
    uint16_t* ucache = reinterpret_cast<uint16_t*>(lds + L.ucache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* go = reinterpret_cast<float*>(lds + L.go);
    float* dz = reinterpret_cast<float*>(lds + L.dz);
    float* zg = reinterpret_cast<float*>(lds + L.z);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, g = lane >> 4;
    const int n = 4 * d;

    for (int j = tid; j < M; j += 256) count[j] = 0;
    for (int q = tid; q < P; q += 256) {
        const int u = unit_idx[q];
        ucache[q] = u >= 0 && u < M ? static_cast<uint16_t>(u) : uint16_t(0xffff);
    }
    __syncthreads();
    for (int q = tid; q < P; q += 256)  // integer counts: any order gives the same
        if (ucache[q] != 0xffff) atomicAdd(&count[ucache[q]], 1);
    __syncthreads();
    if (wave == 0) {
        int unit = -1, tile = 0;
        if (lane == 0) {
            int before = 0;
            for (int j = 0; j < M; ++j) {
                const int t = (count[j] + 15) / 16;
                if (static_cast<int>(blockIdx.x) < before + t) {
                    unit = j;
                    tile = blockIdx.x - before;
                    break;
                }
                before += t;
            }
        }
        unit = __builtin_amdgcn_readfirstlane(unit);
        tile = __builtin_amdgcn_readfirstlane(tile);
        if (lane < 16) rows[lane] = -1;
        if (unit >= 0) {
            const int first = tile * 16;
            int base = 0;
            for (int q0 = 0; q0 < P && base < first + 16; q0 += kWave) {
                const int q = q0 + lane;
                const bool mine = q < P && ucache[q] == unit;
                const uint64_t m = ballot(mine);
                const int rank = base + lanes_below(m);
                if (mine && rank >= first && rank < first + 16) rows[rank - first] = q;
                base += __popcll(m);
            }
        }
        if (lane == 0) meta[0] = unit;
    }
    __syncthreads();
    const int j = meta[0];
    if (j < 0) return;  // past the last tile (uniform)

    const int i0 = blockIdx.y * 64;
    const T* W1j = W1 + int64_t(j) * n * H;
    const T* W2j = W2 + int64_t(j) * H * d;
    const int tiles_h = (H + 63) / 64;
    const int qd = d / 4;  // dz's reduction steps a lane group (d a multiple of 4)
    // the rows' grad_out, widened into LDS
    for (int e = tid; e < 16 * qd; e += 256) {
        const int pp = e / qd, c = 4 * (e % qd);
        const int q = rows[pp];
        const float4 t = q >= 0 ? row4w(grad_out + int64_t(q) * d, c, d, ALIGNED)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float* dst = go + pp * L.sg + c;
        dst[0] = t.x, dst[1] = t.y, dst[2] = t.z, dst[3] = t.w;
    }
    // a hidden tile's fragments: W2[j][h][g qd ..] for this lane's hidden column h (dz), W1[j][i]
    // [h0 + 16 g ..] for its input column i (grad_v), and z1 of 4 (row, h) pairs a thread
    constexpr int kQd = 16;  // dz steps held in registers (d <= 64); beyond, read as they go
    const int hcol = wave * 16 + lr;  // the wavefront's hidden column in the tile
    const int icol = i0 + wave * 16 + lr;
    const bool iin = icol < n;
    struct Frag {
        float w2[kQd];
        float4 w1[4];
        float z[4];
    };
    auto load_frag = [&](Frag& f, int ht) {
        const int h = ht * 64 + hcol;
        const bool hin = h < H;
        const T* w2r = W2j + int64_t(hin ? h : 0) * d + g * qd;
#pragma unroll
        for (int s = 0; s < kQd; s += 4) {
            const float4 t = hin && s < qd ? row4w(w2r, s, qd, ALIGNED)
                                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            f.w2[s] = t.x, f.w2[s + 1] = t.y, f.w2[s + 2] = t.z, f.w2[s + 3] = t.w;
        }
        const T* w1r = W1j + int64_t(iin ? icol : 0) * H + ht * 64 + g * 16;
        const int left = H - (ht * 64 + g * 16);  // this lane group's hidden units in range
#pragma unroll
        for (int s = 0; s < 4; ++s)
            f.w1[s] = iin ? row4w(w1r, 4 * s, left, ALIGNED) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + 256 * u, row = e >> 6, c = e & 63;
            const int q = rows[row];
            f.z[u] = q >= 0 && ht * 64 + c < H ? load_f32(hidden, int64_t(q) * H + ht * 64 + c)
                                               : 0.0f;
        }
    };
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};  // grad_v rows 4 g + r, input column icol
    Frag fa, fb;
    load_frag(fa, 0);
    __syncthreads();  // grad_out is in LDS
    auto tile = [&](int ht, Frag& cur, Frag& nxt) {
        if (ht + 1 < tiles_h) load_frag(nxt, ht + 1);
        // gelu'(z1) of the tile into LDS
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + 256 * u, row = e >> 6, c = e & 63;
            zg[row * 65 + c] = gelu_grad(cur.z[u]);
        }
        // grad_out W2[j]^T for hidden column hcol: A = grad_out rows, B[k][h] = W2[j][h][k]
        v4f t = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* ar = go + lr * L.sg + g * qd;
#pragma unroll
        for (int s = 0; s < kQd; ++s)
            if (s < qd) t = mfma(ar[s], cur.w2[s], t);
        for (int s = kQd; s < qd; ++s) {  // d > 64
            const int h = ht * 64 + hcol;
            const float w = h < H ? load_f32(W2j, int64_t(h) * d + g * qd + s) : 0.0f;
            t = mfma(ar[s], w, t);
        }
        __syncthreads();  // gelu' in LDS
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r;
            dz[row * 65 + hcol] = t[r] * zg[row * 65 + hcol];
        }
        __syncthreads();
        // grad_v += dz1 W1[j]^T: A = dz rows (k = h), B[k][i] = W1[j][i][h0 + k]
        const float* dr = dz + lr * 65 + g * 16;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc = mfma(dr[4 * s], cur.w1[s].x, acc);
            acc = mfma(dr[4 * s + 1], cur.w1[s].y, acc);
            acc = mfma(dr[4 * s + 2], cur.w1[s].z, acc);
            acc = mfma(dr[4 * s + 3], cur.w1[s].w, acc);
        }
        __syncthreads();  // dz and zg are rewritten by the next tile
    };
    for (int ht = 0; ht < tiles_h; ht += 2) {
        tile(ht, fa, fb);
        if (ht + 1 < tiles_h) tile(ht + 1, fb, fa);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int q = rows[4 * g + r];
        if (q >= 0 && iin) store_f32(grad_v, int64_t(q) * n + icol, acc[r]);
    }
}

// ------------------------------------------------------------------------------------------
// csr_messages
// ------------------------------------------------------------------------------------------

struct Csr {
    const int32_t* indptr;   // [N + 1]
    const int32_t* indices;  // [E]
    int N, E;
    // the edge range of row i, clamped into [0, E] (empty for a row outside [0, N))
    __device__ __forceinline__ void range(int i, int& e0, int& e1) const {
        if (i < 0 || i >= N) {
            e0 = e1 = 0;
            return;
        }
        e0 = min(max(indptr[i], 0), E);
        e1 = min(max(indptr[i + 1], e0), E);
    }
};

// S[s][c] = sum_e a[e] h[r_s, indices[e], c] for 16 slots from s0 and columns [c0, c0 + nc),
// into LDS (row stride `ld`); every thread of the workgroup takes (slot, column) pairs and walks
// its slot's edges in order.
template <typename T>
__device__ __forceinline__ void gather_sums(const T* h, const T* a, const int32_t* cell_idx,
                                            const Csr& g, int s0, int BK, int K, int d, int c0,
                                            int nc, float* S, int ld) {
    for (int x = threadIdx.x; x < 16 * nc; x += blockDim.x) {
        const int s = x / nc, cc = x - s * nc;
        const int flat = s0 + s, col = c0 + cc;
        float sum = 0.0f;
        if (flat < BK && col < d) {
            const int r = flat / K;
            int e0, e1;
            g.range(cell_idx[flat], e0, e1);
            for (int e = e0; e < e1; ++e) {
                const int src = g.indices[e];
                if (src >= 0 && src < g.N)
                    sum += load_f32(a, e) * load_f32(h, (int64_t(r) * g.N + src) * d + col);
            }
        }
        S[s * ld + cc] = sum;
    }
}

// S as gather_sums, with the 16 slots' edges listed into LDS first when they fit (kListCap
// entries): wavefront 0 finds the slots' ranges and their offsets, every thread lists entries
// (source, weight), then each (slot, column) sums its slot's entries in edge order with the loads
// of h issued 8 at a time. A longer list takes gather_sums.
constexpr int kListCap = 1024;
// gather_sums_listed's static LDS (the 16 slots' edge list), which counts against the same
// 64 KiB default limit as a caller's dynamic LDS
constexpr size_t kListLds = (17 + 16 + 2 * size_t(kListCap)) * 4;
template <typename T>
__device__ __forceinline__ void gather_sums_listed(const T* h, const T* a,
                                                   const int32_t* cell_idx, const Csr& g, int s0,
                                                   int BK, int K, int d, float* S) {
    __shared__ int lstart[17], le0[16], lsrc[kListCap];
    __shared__ float lw[kListCap];
    const int tid = threadIdx.x, lane = lane_id();
    if (tid < kWave) {
        int e0 = 0, e1 = 0;
        if (lane < 16 && s0 + lane < BK) g.range(cell_idx[s0 + lane], e0, e1);
        int v = lane < 16 ? e1 - e0 : 0;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const int t = __shfl_up(v, off, kWave);
            if (lane >= off) v += t;
        }
        if (lane < 16) {
            le0[lane] = e0;
            lstart[lane + 1] = v;
        }
        if (lane == 0) lstart[0] = 0;
    }
    __syncthreads();
    const int total = lstart[16];
    if (total > kListCap) {  // uniform
        gather_sums<T>(h, a, cell_idx, g, s0, BK, K, d, 0, d, S, d);
        return;
    }
    for (int x = tid; x < total; x += blockDim.x) {
        int lo = 0, hi = 16;  // lstart[lo] <= x < lstart[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (lstart[mid] <= x) lo = mid;
            else hi = mid;
        }
        const int e = le0[lo] + x - lstart[lo];
        const int src = g.indices[e];
        lsrc[x] = src >= 0 && src < g.N ? src : -1;
        lw[x] = load_f32(a, e);
    }
    __syncthreads();
    for (int x = tid; x < 16 * d; x += blockDim.x) {
        const int sl = x / d, col = x - sl * d;
        const int flat = s0 + sl;
        float sum = 0.0f;
        if (flat < BK) {
            const T* hr = h + int64_t(flat / K) * g.N * d + col;
            const int b0 = lstart[sl], b1 = lstart[sl + 1];
            for (int j0 = b0; j0 < b1; j0 += 8) {
                float hv[8], wv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int src = j0 + u < b1 ? lsrc[j0 + u] : -1;
                    wv[u] = src >= 0 ? lw[j0 + u] : 0.0f;
                    hv[u] = src >= 0 ? load_f32(hr, int64_t(src) * d) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (j0 + u < b1 && lsrc[j0 + u] >= 0) sum += wv[u] * hv[u];
            }
        }
        S[x] = sum;
    }
}

// (BK / 16, d / 64) workgroups: m[s][o] = sum_c V[o][c] S[s][c] for 16 slots (S in LDS).
template <typename T>
__global__ __launch_bounds__(256) void csr_fwd(const T* h, const Csr g, const T* a, const T* V,
                                               const int32_t* cell_idx, T* m, int B, int K,
                                               int d) {
    extern __shared__ float S[];  // [16][d]
    const int lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15, lq = lane >> 4;
    const int BK = B * K, s0 = blockIdx.x * 16;
    gather_sums_listed<T>(h, a, cell_idx, g, s0, BK, K, d, S);
    __syncthreads();
    const int o = blockIdx.y * 64 + 16 * w + lr;
    const bool oin = o < d;
    const T* Vr = V + int64_t(oin ? o : 0) * d;  // B[c][o] = V[o][c]
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < d; k0 += 4) {
        const int k = k0 + lq;
        const float av = k < d ? S[lr * d + k] : 0.0f;
        const float bv = oin && k < d ? load_f32(Vr, k) : 0.0f;
        acc = mfma(av, bv, acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int flat = s0 + 4 * lq + r;
        if (flat < BK && oin) store_f32(m, int64_t(flat) * d + o, acc[r]);
    }
}

// (B, d / 64) wavefronts: row r's grad_h for 64 columns, one lane per column, in blocks of
// kDhCells source cells accumulated in LDS: every slot in order adds a[e] (V^T grad_m[r, k])[c]
// to the source cell of each of its edges, in edge order, so every sum has a fixed order.
constexpr int kDhCells = 128;
template <typename T>
__global__ __launch_bounds__(64) void csr_dh(const Csr g, const T* a, const T* V,
                                             const int32_t* cell_idx, const T* grad_m, T* grad_h,
                                             int K, int d) {
    __shared__ float acc[kDhCells][64];
    const int r = blockIdx.x, lane = lane_id(), c = blockIdx.y * 64 + lane;
    const bool cin = c < d;
    T* gh = grad_h + int64_t(r) * g.N * d;
    for (int n0 = 0; n0 < g.N; n0 += kDhCells) {
        for (int n = 0; n < kDhCells; ++n) acc[n][lane] = 0.0f;
        for (int k = 0; k < K; ++k) {
            const int flat = r * K + k;
            int e0, e1;
            g.range(cell_idx[flat], e0, e1);
            bool any = false;  // an edge of this slot with its source in the block
            for (int e = e0; e < e1 && !any; ++e) {
                const int src = g.indices[e];
                any = src >= n0 && src < n0 + kDhCells && src < g.N;
            }
            if (!any) continue;
            float u = 0.0f;  // (V^T grad_m[r, k])[c]
            if (cin)
                for (int o = 0; o < d; ++o)
                    u += load_f32(V, int64_t(o) * d + c) * load_f32(grad_m, int64_t(flat) * d + o);
            for (int e = e0; e < e1; ++e) {
                const int src = g.indices[e];
                if (src >= n0 && src < n0 + kDhCells && src < g.N)
                    acc[src - n0][lane] += load_f32(a, e) * u;
            }
        }
        if (cin)
            for (int n = n0; n < min(g.N, n0 + kDhCells); ++n)
                store_f32(gh, int64_t(n) * d + c, acc[n - n0][lane]);
    }
}

// A wavefront per edge e (target row i, source j): grad_a[e] = sum over the slots (r, k) that
// selected row i, in order, of grad_m[r, k] . (V h[r, j]).
template <typename T>
__global__ __launch_bounds__(256) void csr_da(const T* h, const Csr g, const T* V,
                                              const int32_t* cell_idx, const T* grad_m, T* grad_a,
                                              int B, int K, int d) {
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = lane_id();
    if (e >= g.E) return;
    // the target row: the last i with indptr[i] <= e (binary search; a malformed CSR may give
    // a row whose range excludes e, which then contributes nothing)
    int lo = 0, hi = g.N;  // indptr[lo] <= e < indptr[hi] when well formed
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (g.indptr[mid] <= e) lo = mid;
        else hi = mid;
    }
    int e0, e1;
    g.range(lo, e0, e1);
    const int src = g.indices[e];
    float acc = 0.0f;
    if (e >= e0 && e < e1 && src >= 0 && src < g.N) {
        for (int flat = 0; flat < B * K; ++flat) {
            if (cell_idx[flat] != lo) continue;  // uniform
            const int r = flat / K;
            const T* hr = h + (int64_t(r) * g.N + src) * d;
            const T* gm = grad_m + int64_t(flat) * d;
            for (int o = lane; o < d; o += 64) {  // lane o: grad_m[o] (V h)[o]
                float vh = 0.0f;
                for (int cc = 0; cc < d; ++cc) vh += load_f32(V, int64_t(o) * d + cc) * load_f32(hr, cc);
                acc += load_f32(gm, o) * vh;
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    if (lane == 0) store_f32(grad_a, e, acc);
}


// grad_h by (row, 64 columns, 128 source cells) workgroups with the row's work staged in LDS
// (K <= 64). u[k] = V^T grad_m[r, k] comes first, for the 64 columns, through LDS blocks of 64
// rows of V; then the row's edges in slot and edge order (source, weight, slot) are listed into
// LDS kDhList at a time, each wavefront owns 32 of the 128 cells and walks the whole list, adding
// a[e] u[k] to the cells it owns, so every cell's sum keeps the list's order. Cells no edge names
// get zeros.
constexpr int kDhList = 1024;
struct DhLds {
    int start, e0, u, src, w, slot, acc, bytes;
};
__host__ __device__ inline DhLds dh_lds(int K) {
    DhLds L;
    L.start = 0;                                // int [K + 1]
    L.e0 = L.start + 4 * (K + 1);               // int [K]
    L.u = (L.e0 + 4 * K + 15) & ~15;            // float [K][64]
    L.src = L.u + 4 * 64 * K;                   // int [kDhList]
    L.w = L.src + 4 * kDhList;                  // float [kDhList]
    L.slot = L.w + 4 * kDhList;                 // int [kDhList]
    L.acc = L.slot + 4 * kDhList;               // float [128][64]; first V's block and grad_m's
    const int stage = 4 * (64 * 64 + 64 * K);   // [64][64] and [K][64]
    L.bytes = L.acc + (stage > 4 * 128 * 64 ? stage : 4 * 128 * 64);
    return L;
}

template <typename T>
__global__ __launch_bounds__(256) void csr_dh_rows(const Csr g, const T* a, const T* V,
                                                   const int32_t* cell_idx, const T* grad_m,
                                                   T* grad_h, int K, int d) {
    extern __shared__ __align__(16) unsigned char lds[];
    const DhLds L = dh_lds(K);
    int* start = reinterpret_cast<int*>(lds + L.start);
    int* se0 = reinterpret_cast<int*>(lds + L.e0);
    float* u = reinterpret_cast<float*>(lds + L.u);
    int* lsrc = reinterpret_cast<int*>(lds + L.src);
    float* lw = reinterpret_cast<float*>(lds + L.w);
    int* lslot = reinterpret_cast<int*>(lds + L.slot);
    float* acc = reinterpret_cast<float*>(lds + L.acc);
    float* Vs = acc;            // [64 rows o][64 columns]
    float* gs = acc + 64 * 64;  // [K][64 rows o]
    const int r = blockIdx.x, c0 = blockIdx.y * 64, n0 = blockIdx.z * 128;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // the first block of V's rows and of grad_m's values in flight during the slots' scan
    float vpre[16], gpre[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int x = tid + 256 * i, oo = x >> 6, cc = x & 63;
        vpre[i] = oo < d && c0 + cc < d ? load_f32(V, int64_t(oo) * d + c0 + cc) : 0.0f;
        gpre[i] = x < K * 64 && cc < d ? load_f32(grad_m, (int64_t(r) * K + oo) * d + cc) : 0.0f;
    }
    // the slots' edge ranges and their offsets in the list (an inclusive scan in wavefront 0)
    if (wave == 0) {
        int e0 = 0, e1 = 0;
        if (lane < K) g.range(cell_idx[r * K + lane], e0, e1);
        int v = e1 - e0;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(v, off, kWave);
            if (lane >= off) v += t;
        }
        if (lane < K) {
            se0[lane] = e0;
            start[lane + 1] = v;
        }
        if (lane == 0) start[0] = 0;
    }
    for (int x = tid; x < K * 64; x += 256) u[x] = 0.0f;
    for (int o0 = 0; o0 < d; o0 += 64) {
        __syncthreads();
        if (o0 == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int x = tid + 256 * i;
                Vs[x] = vpre[i];
                if (x < K * 64) gs[x] = gpre[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int x = tid + 256 * i, oo = x >> 6, cc = x & 63;
                Vs[x] = o0 + oo < d && c0 + cc < d ? load_f32(V, int64_t(o0 + oo) * d + c0 + cc)
                                                   : 0.0f;
            }
            for (int x = tid; x < K * 64; x += 256) {
                const int k = x >> 6, oo = x & 63;
                gs[x] = o0 + oo < d ? load_f32(grad_m, (int64_t(r) * K + k) * d + o0 + oo) : 0.0f;
            }
        }
        __syncthreads();
        for (int x = tid; x < K * 64; x += 256) {  // the same thread owns u[x] every block
            const int k = x >> 6, cc = x & 63;
            float sum = u[x];
#pragma unroll 8
            for (int oo = 0; oo < 64; ++oo) sum += Vs[oo * 64 + cc] * gs[k * 64 + oo];
            u[x] = sum;
        }
    }
    __syncthreads();
    const int total = start[K];
    const int lo = n0 + 32 * wave, hi = min(lo + 32, g.N);
    for (int n = lo; n < hi; ++n) acc[(n - n0) * 64 + lane] = 0.0f;
    for (int p0 = 0; p0 < total; p0 += kDhList) {
        const int cnt = min(kDhList, total - p0);
        __syncthreads();  // the last block's walk is done
        for (int x = tid; x < cnt; x += 256) {
            const int pos = p0 + x;
            int klo = 0, khi = K;  // start[klo] <= pos < start[khi]
            while (khi - klo > 1) {
                const int mid = (klo + khi) >> 1;
                if (start[mid] <= pos) klo = mid;
                else khi = mid;
            }
            const int e = se0[klo] + pos - start[klo];
            const int src = g.indices[e];
            lsrc[x] = src >= n0 && src < min(n0 + 128, g.N) ? src : -1;
            lw[x] = load_f32(a, e);
            lslot[x] = klo;
        }
        __syncthreads();
        for (int i0 = 0; i0 < cnt; i0 += 64) {  // 64 entries a lane, broadcast in order
            const int m = min(64, cnt - i0);
            const int my_src = lane < m ? lsrc[i0 + lane] : -1;
            const int my_w = lane < m ? __float_as_int(lw[i0 + lane]) : 0;
            const int my_slot = lane < m ? lslot[i0 + lane] : 0;
            for (int t = 0; t < m; ++t) {
                const int src = __builtin_amdgcn_readlane(my_src, t);
                if (src >= lo && src < hi) {  // uniform
                    const float wt = __int_as_float(__builtin_amdgcn_readlane(my_w, t));
                    const int sl = __builtin_amdgcn_readlane(my_slot, t);
                    acc[(src - n0) * 64 + lane] += wt * u[sl * 64 + lane];
                }
            }
        }
    }
    const int c = c0 + lane;
    if (c < d) {
        T* gh = grad_h + int64_t(r) * g.N * d;
        for (int n = lo; n < hi; ++n) store_f32(gh, int64_t(n) * d + c, acc[(n - n0) * 64 + lane]);
    }
}

// grad_V by groups of slots, (group, 16 columns, 64 rows) workgroups: the group's slots in
// chunks of 16, S[s][c] = sum_e a[e] h[r_s, indices[e], c] gathered a (slot, column) a thread into
// LDS, then grad_m[s]^T S[s] on MFMA, wavefront w taking rows o0 + 16 w .. + 16. With one group
// the sum goes straight to grad_V; with more, each group's [d][d] fp32 sum goes to part[group]
// and csr_dV_sum adds the groups in order.
template <typename T>
__global__ __launch_bounds__(256) void csr_dV_groups(const T* h, const Csr g, const T* a,
                                                     const int32_t* cell_idx, const T* grad_m,
                                                     T* grad_V, float* part, int B, int K, int d,
                                                     int group_slots) {
    __shared__ float S[16 * 16];
    const int lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15, lq = lane >> 4;
    const int BK = B * K;
    const int sb = blockIdx.x * group_slots, se = min(BK, sb + group_slots);
    const int c0 = blockIdx.y * 16, o = blockIdx.z * 64 + 16 * w + lr;
    const int s = threadIdx.x >> 4, cc = threadIdx.x & 15;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = sb; s0 < se; s0 += 16) {
        const int flat = s0 + s, col = c0 + cc;
        float sum = 0.0f;
        if (flat < se && col < d) {
            const int r = flat / K;
            int e0, e1;
            g.range(cell_idx[flat], e0, e1);
            const T* hr = h + int64_t(r) * g.N * d + col;
#pragma unroll 4
            for (int e = e0; e < e1; ++e) {
                const int src = g.indices[e];
                if (src >= 0 && src < g.N) sum += load_f32(a, e) * load_f32(hr, int64_t(src) * d);
            }
        }
        __syncthreads();  // the last chunk's products are done
        S[threadIdx.x] = sum;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = 4 * q + lq;
            const float av = s0 + k < se && o < d ? load_f32(grad_m, int64_t(s0 + k) * d + o) : 0.0f;
            acc = mfma(av, S[k * 16 + lr], acc);
        }
    }
    const int c = c0 + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int orow = blockIdx.z * 64 + 16 * w + 4 * lq + i;
        if (orow < d && c < d) {
            if (part) part[int64_t(blockIdx.x) * d * d + int64_t(orow) * d + c] = acc[i];
            else store_f32(grad_V, int64_t(orow) * d + c, acc[i]);
        }
    }
}

// U[s][c] = sum_o grad_m[s][o] V[o][c] for 16 slots and 64 columns a workgroup (MFMA, wavefront
// w taking columns c0 + 16 w .. + 16), in fp32 for csr_da_u.
template <typename T>
__global__ __launch_bounds__(256) void csr_u(const T* V, const T* grad_m, float* U, int BK,
                                             int d) {
    const int lane = lane_id(), w = threadIdx.x >> 6, lr = lane & 15, lq = lane >> 4;
    const int s0 = blockIdx.x * 16, c = blockIdx.y * 64 + 16 * w + lr;
    const bool sin = s0 + lr < BK, cin = c < d;
    const T* gm = grad_m + int64_t(sin ? s0 + lr : 0) * d;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int o0 = 0; o0 < d; o0 += 4) {
        const int o = o0 + lq;
        const float av = sin && o < d ? load_f32(gm, o) : 0.0f;
        const float bv = cin && o < d ? load_f32(V, int64_t(o) * d + c) : 0.0f;
        acc = mfma(av, bv, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = s0 + 4 * lq + i;
        if (s < BK && cin) U[int64_t(s) * d + c] = acc[i];
    }
}

// grad_a from U: a wavefront per edge e (target row i, source j) adds U[r, k] . h[r, j] over the
// slots that selected row i, in order. The slots' cells and indptr are staged in LDS
// ((B K + N + 1) ints within 64 KiB); the slots are found 64 at a time by a ballot and taken in
// ascending order from its set bits.
template <typename T>
__global__ __launch_bounds__(256) void csr_da_u(const T* h, const Csr g, const float* U,
                                                const int32_t* cell_idx, T* grad_a, int B, int K,
                                                int d) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int BK = B * K;
    int* cells = reinterpret_cast<int*>(lds);
    int* ptr = cells + BK;
    for (int x = threadIdx.x; x < BK; x += 256) cells[x] = cell_idx[x];
    for (int x = threadIdx.x; x <= g.N; x += 256) ptr[x] = g.indptr[x];
    __syncthreads();
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = lane_id();
    if (e >= g.E) return;
    int lo = 0, hi = g.N;  // the target row: the last i with indptr[i] <= e
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (ptr[mid] <= e) lo = mid;
        else hi = mid;
    }
    const int e0 = min(max(ptr[lo], 0), g.E), e1 = min(max(ptr[lo + 1], e0), g.E);
    const int src = g.indices[e];
    float acc = 0.0f;
    if (e >= e0 && e < e1 && src >= 0 && src < g.N) {
        for (int f0 = 0; f0 < BK; f0 += 64) {
            uint64_t hits = ballot(f0 + lane < BK && cells[f0 + lane] == lo);
            while (hits) {  // uniform
                const int flat = f0 + __builtin_ctzll(hits);
                hits &= hits - 1;
                const T* hr = h + (int64_t(flat / K) * g.N + src) * d;
                const float* u = U + int64_t(flat) * d;
                for (int c = lane; c < d; c += 64) acc += u[c] * load_f32(hr, c);
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    if (lane == 0) store_f32(grad_a, e, acc);
}

template <typename T>
__global__ __launch_bounds__(256) void csr_dV_sum(const float* part, T* grad_V, int groups, int dd) {
    const int x = blockIdx.x * 256 + threadIdx.x;
    if (x >= dd) return;
    float sum = 0.0f;  // the loads issued 8 at a time; the sum keeps the groups' order
#pragma unroll 8
    for (int i = 0; i < groups; ++i) sum += part[int64_t(i) * dd + x];
    store_f32(grad_V, x, sum);
}

// grad_a with the slots' cells staged in LDS (B K <= 16384): a wavefront per edge e (target row
// i, source j) finds the slots that selected row i in the LDS copy, in order, and adds
// (V^T grad_m[r, k]) . h[r, j] for each, lane c taking column c (then a wavefront sum).
template <typename T>
__global__ __launch_bounds__(256) void csr_da_rows(const T* h, const Csr g, const T* V,
                                                   const int32_t* cell_idx, const T* grad_m,
                                                   T* grad_a, int B, int K, int d) {
    extern __shared__ __align__(16) unsigned char lds[];
    int* cells = reinterpret_cast<int*>(lds);
    const int BK = B * K;
    for (int x = threadIdx.x; x < BK; x += 256) cells[x] = cell_idx[x];
    __syncthreads();
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = lane_id();
    if (e >= g.E) return;
    int lo = 0, hi = g.N;  // the target row: the last i with indptr[i] <= e
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (g.indptr[mid] <= e) lo = mid;
        else hi = mid;
    }
    int e0, e1;
    g.range(lo, e0, e1);
    const int src = g.indices[e];
    float acc = 0.0f;
    if (e >= e0 && e < e1 && src >= 0 && src < g.N) {
        for (int flat = 0; flat < BK; ++flat) {
            if (cells[flat] != lo) continue;  // uniform
            const int r = flat / K;
            const T* hr = h + (int64_t(r) * g.N + src) * d;
            const T* gm = grad_m + int64_t(flat) * d;
            for (int c = lane; c < d; c += 64) {  // lane c: (V^T grad_m)[c] h[c]
                float ug = 0.0f;
#pragma unroll 8
                for (int o = 0; o < d; ++o) ug += load_f32(V, int64_t(o) * d + c) * load_f32(gm, o);
                acc += ug * load_f32(hr, c);
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    if (lane == 0) store_f32(grad_a, e, acc);
}
}  // namespace units
}  // namespace hsn

using namespace hsn;

namespace {

template <template <typename> class Fn, typename... Args>
void by_dtype(int dtype, Args&&... args) {
    if (dtype == HSN_DTYPE_F32) Fn<float>::run(args...);
    else if (dtype == HSN_DTYPE_F16) Fn<_Float16>::run(args...);
    else Fn<bf16_t>::run(args...);
}

void check_dtype(int dtype, const char* who) {
    HSN_REQUIRE(dtype == HSN_DTYPE_F32 || dtype == HSN_DTYPE_F16 || dtype == HSN_DTYPE_BF16,
                HSN_ERR_UNSUPPORTED_DTYPE, std::string(who) + ": unknown dtype code");
}

void check_units(int P, int M, int d, int H, const char* who) {
    HSN_REQUIRE(P >= 1 && M >= 1 && d >= 1 && H >= 1, HSN_ERR_INVALID_ARGUMENT,
                std::string(who) + ": dimensions must be >= 1");
    HSN_REQUIRE(d <= 256, HSN_ERR_INVALID_ARGUMENT, std::string(who) + ": d above 256");
    HSN_REQUIRE(int64_t(M) * 4 * d * H <= INT32_MAX && int64_t(P) * H <= INT32_MAX &&
                    int64_t(P) * 4 * d <= INT32_MAX,
                HSN_ERR_SIZE_OVERFLOW, std::string(who) + ": an element count exceeds INT32_MAX");
}

void check_csr(int B, int N, int d, int K, int E, const char* who) {
    HSN_REQUIRE(B >= 1 && N >= 1 && d >= 1 && K >= 1 && E >= 0, HSN_ERR_INVALID_ARGUMENT,
                std::string(who) + ": dimensions must be >= 1 (E >= 0)");
    HSN_REQUIRE(d <= 1024, HSN_ERR_INVALID_ARGUMENT, std::string(who) + ": d above 1024");
    HSN_REQUIRE(int64_t(B) * N * d <= INT32_MAX && int64_t(B) * K * d <= INT32_MAX &&
                    int64_t(d) * d <= INT32_MAX && N < INT32_MAX,
                HSN_ERR_SIZE_OVERFLOW, std::string(who) + ": an element count exceeds INT32_MAX");
}

inline dim3 tiles(int n, int per) { return dim3((n + per - 1) / per); }

template <typename T>
struct RunMlp {
    static void run(const void* v, const int32_t* idx, const void* W1, const void* b1,
                    const void* W2, const void* b2, void* hidden, void* out, int P, int M, int d,
                    int H, hipStream_t st) {
        if (d % 4 == 0 && P <= units::kTileMaxSlots && M <= units::kTileMaxUnits &&
            units::tile_lds(P, M, d, H).bytes <= 160 * 1024) {
            const int lds = units::tile_lds(P, M, d, H).bytes;
            auto launch = [&](auto kernel) {
                if (lds > 64 * 1024)
                    HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(kernel), lds));
                hipLaunchKernelGGL(kernel, dim3((P + 15) / 16 + M), dim3(256), lds, st,
                                   static_cast<const T*>(v), idx, static_cast<const T*>(W1),
                                   static_cast<const T*>(b1), static_cast<const T*>(W2),
                                   static_cast<const T*>(b2), static_cast<T*>(hidden),
                                   static_cast<T*>(out), P, M, d, H);
            };
            const int olds = units::out_lds(P, M, H).bytes;
            if (sizeof(T) == 4 && olds <= 160 * 1024) {
                // fp32 storage: the hidden layer over (row tile, hidden tile) workgroups, then
                // the second layer from the stored z1
                auto kernel = H % 4 == 0 ? &units::mlp_fwd_tiles<T, true, true>
                                         : &units::mlp_fwd_tiles<T, false, true>;
                if (lds > 64 * 1024)
                    HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(kernel), lds));
                hipLaunchKernelGGL(kernel, dim3((P + 15) / 16 + M, (H + 63) / 64), dim3(256), lds,
                                   st, static_cast<const T*>(v), idx, static_cast<const T*>(W1),
                                   static_cast<const T*>(b1), static_cast<const T*>(W2),
                                   static_cast<const T*>(b2), static_cast<T*>(hidden),
                                   static_cast<T*>(out), P, M, d, H);
                auto second = &units::mlp_out_tiles<T>;
                if (olds > 64 * 1024)
                    HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(second), olds));
                hipLaunchKernelGGL(second, dim3((P + 15) / 16 + M, (d + 15) / 16), dim3(256), olds,
                                   st, idx,
                                   static_cast<const T*>(W2), static_cast<const T*>(b2),
                                   static_cast<const T*>(hidden), static_cast<T*>(out), P, M, d,
                                   H);
                return;
            }
            if (H % 4 == 0) launch(&units::mlp_fwd_tiles<T, true>);
            else launch(&units::mlp_fwd_tiles<T, false>);
            return;
        }
        const int S = std::min((P + 15) / 16, 64);  // chunk slots per unit
        hipLaunchKernelGGL((units::mlp_fwd<T>), dim3(M, S), dim3(256), 0, st,
                           static_cast<const T*>(v), idx, static_cast<const T*>(W1),
                           static_cast<const T*>(b1), static_cast<const T*>(W2),
                           static_cast<const T*>(b2), static_cast<T*>(hidden),
                           static_cast<T*>(out), P, d, H);
    }
};

template <typename T>
struct RunMlpBwd {
    static void run(const void* v, const int32_t* idx, const void* W1, const void* W2,
                    const void* hidden, const void* dout, void* dv, void* dW1, void* db1,
                    void* dW2, void* db2, int P, int M, int d, int H, hipStream_t st) {
        // grad_v through dz1 in fp32 in grad_W2's memory (4-byte aligned, P H floats of room),
        // before the weight-gradient kernel writes grad_W2
        const int dzl = units::dz_lds(P, M, d).bytes, gvl = units::gv_lds(P, M, H).bytes;
        if (d % 4 == 0 && P <= units::kTileMaxSlots && M <= units::kTileMaxUnits &&
            reinterpret_cast<uintptr_t>(dW2) % 4 == 0 &&
            int64_t(M) * H * d * int64_t(sizeof(T)) >= int64_t(P) * H * 4 && dzl <= 160 * 1024 &&
            gvl <= 160 * 1024) {
            float* dz = static_cast<float*>(dW2);
            auto k1 = &units::mlp_dz_tiles<T>;
            if (dzl > 64 * 1024) HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(k1), dzl));
            hipLaunchKernelGGL(k1, dim3((P + 15) / 16 + M, (H + 63) / 64), dim3(256), dzl, st, idx,
                               static_cast<const T*>(W2), static_cast<const T*>(hidden),
                               static_cast<const T*>(dout), dz, P, M, d, H);
            auto k2 = &units::mlp_gv_tiles<T>;
            if (gvl > 64 * 1024) HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(k2), gvl));
            hipLaunchKernelGGL(k2, dim3((P + 15) / 16 + M, (4 * d + 15) / 16), dim3(256), gvl, st,
                               idx, static_cast<const T*>(W1), static_cast<const float*>(dz),
                               static_cast<T*>(dv), P, M, d, H);
            hipLaunchKernelGGL((units::mlp_dw<T>), dim3((H + 63) / 64, M, (4 * d + 63) / 64),
                               dim3(256), 0, st, static_cast<const T*>(v), idx,
                               static_cast<const T*>(W2), static_cast<const T*>(hidden),
                               static_cast<const T*>(dout), static_cast<T*>(dW1),
                               static_cast<T*>(db1), static_cast<T*>(dW2), static_cast<T*>(db2),
                               P, d, H);
            return;
        }
        hipLaunchKernelGGL((units::mlp_dw<T>), dim3((H + 63) / 64, M, (4 * d + 63) / 64),
                           dim3(256), 0, st, static_cast<const T*>(v), idx,
                           static_cast<const T*>(W2), static_cast<const T*>(hidden),
                           static_cast<const T*>(dout), static_cast<T*>(dW1),
                           static_cast<T*>(db1), static_cast<T*>(dW2), static_cast<T*>(db2), P, d,
                           H);
        if (d % 4 == 0 && P <= units::kTileMaxSlots && M <= units::kTileMaxUnits &&
            units::dv_lds(P, M, d).bytes <= 160 * 1024) {
            const int lds = units::dv_lds(P, M, d).bytes;
            auto launch = [&](auto kernel) {
                if (lds > 64 * 1024)
                    HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(kernel), lds));
                hipLaunchKernelGGL(kernel, dim3((P + 15) / 16 + M, (4 * d + 63) / 64), dim3(256),
                                   lds, st, idx, static_cast<const T*>(W1),
                                   static_cast<const T*>(W2), static_cast<const T*>(hidden),
                                   static_cast<const T*>(dout), static_cast<T*>(dv), P, M, d, H);
            };
            if (H % 4 == 0 && d % 16 == 0) launch(&units::mlp_dv_tiles<T, true>);
            else launch(&units::mlp_dv_tiles<T, false>);
            return;
        }
        hipLaunchKernelGGL((units::mlp_dv<T>), dim3((4 * d + 63) / 64, M), dim3(256), 0, st, idx,
                           static_cast<const T*>(W1), static_cast<const T*>(W2),
                           static_cast<const T*>(hidden), static_cast<const T*>(dout),
                           static_cast<T*>(dv), P, d, H);
    }
};

template <typename T>
struct RunCsr {
    static void run(const void* h, const int32_t* indptr, const int32_t* indices, const void* a,
                    const void* V, const int32_t* idx, void* m, int B, int N, int d, int K, int E,
                    hipStream_t st) {
        const units::Csr g{indptr, indices, N, E};
        // S [16][d] in dynamic LDS beside the static edge list: above the default 64 KiB from
        // d = 894 on (d <= 1024: at most 72.3 KiB of the CU's 160)
        const size_t lds = size_t(16) * d * 4;
        if (lds + units::kListLds > 64 * 1024)
            HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(units::csr_fwd<T>), lds));
        hipLaunchKernelGGL((units::csr_fwd<T>), dim3((B * K + 15) / 16, (d + 63) / 64),
                           dim3(256), lds, st, static_cast<const T*>(h), g,
                           static_cast<const T*>(a), static_cast<const T*>(V), idx,
                           static_cast<T*>(m), B, K, d);
    }
};

template <typename T>
struct RunCsrBwd {
    static void run(const void* h, const int32_t* indptr, const int32_t* indices, const void* a,
                    const void* V, const int32_t* idx, const void* dm, void* dh, void* da,
                    void* dV, int B, int N, int d, int K, int E, hipStream_t st) {
        const units::Csr g{indptr, indices, N, E};
        // grad_V first: with more than one group of slots its fp32 partial sums live in grad_h's
        // memory (4-byte aligned and large enough), which the grad_h kernel then overwrites
        const int BK = B * K, chunks = (BK + 15) / 16;
        const int64_t room = reinterpret_cast<uintptr_t>(dh) % 4 == 0
                                 ? int64_t(B) * N * d * int64_t(sizeof(T)) / (int64_t(d) * d * 4)
                                 : 0;
        int groups = 1, group_slots = 16 * chunks;
        if (chunks > 1 && room >= 2) {
            const int most = static_cast<int>(std::min<int64_t>(room, 256));
            group_slots = 16 * ((chunks + most - 1) / most);
            groups = (BK + group_slots - 1) / group_slots;
        }
        float* part = groups > 1 ? static_cast<float*>(dh) : nullptr;
        hipLaunchKernelGGL((units::csr_dV_groups<T>), dim3(groups, (d + 15) / 16, (d + 63) / 64),
                           dim3(256), 0, st, static_cast<const T*>(h), g,
                           static_cast<const T*>(a), idx, static_cast<const T*>(dm),
                           static_cast<T*>(dV), part, B, K, d, group_slots);
        if (part)
            hipLaunchKernelGGL((units::csr_dV_sum<T>), dim3((d * d + 255) / 256), dim3(256), 0, st,
                               part, static_cast<T*>(dV), groups, d * d);
        // grad_a next, from U = grad_m V in grad_h's memory when it fits there
        const bool u_fits = reinterpret_cast<uintptr_t>(dh) % 4 == 0 &&
                            int64_t(BK) * d * 4 <= int64_t(B) * N * d * int64_t(sizeof(T));
        if (E > 0 && int64_t(BK) + N + 1 <= 16384 && u_fits) {
            float* U = static_cast<float*>(dh);
            hipLaunchKernelGGL((units::csr_u<T>), dim3(chunks, (d + 63) / 64), dim3(256), 0, st,
                               static_cast<const T*>(V), static_cast<const T*>(dm), U, BK, d);
            hipLaunchKernelGGL((units::csr_da_u<T>), dim3((E + 3) / 4), dim3(256),
                               size_t(4) * (BK + N + 1),
                               st, static_cast<const T*>(h), g, U, idx, static_cast<T*>(da), B,
                               K, d);
        } else if (E > 0 && BK <= 16384) {
            hipLaunchKernelGGL((units::csr_da_rows<T>), dim3((E + 3) / 4), dim3(256),
                               size_t(4) * BK, st, static_cast<const T*>(h), g,
                               static_cast<const T*>(V), idx, static_cast<const T*>(dm),
                               static_cast<T*>(da), B, K, d);
        } else if (E > 0) {
            hipLaunchKernelGGL((units::csr_da<T>), dim3((E + 3) / 4), dim3(256), 0, st,
                               static_cast<const T*>(h), g, static_cast<const T*>(V), idx,
                               static_cast<const T*>(dm), static_cast<T*>(da), B, K, d);
        }
        if (K <= 64)
            hipLaunchKernelGGL((units::csr_dh_rows<T>), dim3(B, (d + 63) / 64, (N + 127) / 128),
                               dim3(256), units::dh_lds(K).bytes, st, g, static_cast<const T*>(a),
                               static_cast<const T*>(V), idx, static_cast<const T*>(dm),
                               static_cast<T*>(dh), K, d);
        else
            hipLaunchKernelGGL((units::csr_dh<T>), dim3(B, (d + 63) / 64), dim3(64), 0, st, g,
                               static_cast<const T*>(a), static_cast<const T*>(V), idx,
                               static_cast<const T*>(dm), static_cast<T*>(dh), K, d);
    }
};

}  // namespace

extern "C" int hsn_grouped_unit_mlp_fwd(const void* v, const int32_t* unit_idx, const void* W1,
                                        const void* b1, const void* W2, const void* b2,
                                        void* hidden_saved, void* out, int P, int M, int d, int H,
                                        int dtype, void* stream) {
    HSN_ABI_BEGIN
    check_units(P, M, d, H, "hsn_grouped_unit_mlp_fwd");
    check_dtype(dtype, "hsn_grouped_unit_mlp_fwd");
    HSN_REQUIRE(v && unit_idx && W1 && b1 && W2 && b2 && hidden_saved && out,
                HSN_ERR_INVALID_ARGUMENT, "hsn_grouped_unit_mlp_fwd: a pointer is NULL");
    by_dtype<RunMlp>(dtype, v, unit_idx, W1, b1, W2, b2, hidden_saved, out, P, M, d, H,
                     as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_grouped_unit_mlp_bwd(const void* v, const int32_t* unit_idx, const void* W1,
                                        const void* W2, const void* hidden_saved,
                                        const void* grad_out, void* grad_v, void* grad_W1,
                                        void* grad_b1, void* grad_W2, void* grad_b2, int P, int M,
                                        int d, int H, int dtype, int deterministic,
                                        void* stream) {
    HSN_ABI_BEGIN
    check_units(P, M, d, H, "hsn_grouped_unit_mlp_bwd");
    check_dtype(dtype, "hsn_grouped_unit_mlp_bwd");
    HSN_REQUIRE(deterministic == 0 || deterministic == 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_grouped_unit_mlp_bwd: deterministic must be 0 or 1");
    HSN_REQUIRE(v && unit_idx && W1 && W2 && hidden_saved && grad_out && grad_v && grad_W1 &&
                    grad_b1 && grad_W2 && grad_b2,
                HSN_ERR_INVALID_ARGUMENT, "hsn_grouped_unit_mlp_bwd: a pointer is NULL");
    HSN_REQUIRE(M <= 65535, HSN_ERR_INVALID_ARGUMENT, "hsn_grouped_unit_mlp_bwd: M above 65535");
    by_dtype<RunMlpBwd>(dtype, v, unit_idx, W1, W2, hidden_saved, grad_out, grad_v, grad_W1,
                        grad_b1, grad_W2, grad_b2, P, M, d, H, as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_csr_messages(const void* h, const int32_t* indptr, const int32_t* indices,
                                const void* a, const void* V, const int32_t* cell_idx, void* m,
                                int B, int N, int d, int K, int E, int dtype, void* stream) {
    HSN_ABI_BEGIN
    check_csr(B, N, d, K, E, "hsn_csr_messages");
    check_dtype(dtype, "hsn_csr_messages");
    HSN_REQUIRE(h && indptr && V && cell_idx && m && (E == 0 || (indices && a)),
                HSN_ERR_INVALID_ARGUMENT, "hsn_csr_messages: a pointer is NULL");
    by_dtype<RunCsr>(dtype, h, indptr, indices, a, V, cell_idx, m, B, N, d, K, E,
                     as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}

extern "C" int hsn_csr_messages_bwd(const void* h, const int32_t* indptr, const int32_t* indices,
                                    const void* a, const void* V, const int32_t* cell_idx,
                                    const void* grad_m, void* grad_h, void* grad_a, void* grad_V,
                                    int B, int N, int d, int K, int E, int dtype,
                                    int deterministic, void* stream) {
    HSN_ABI_BEGIN
    check_csr(B, N, d, K, E, "hsn_csr_messages_bwd");
    check_dtype(dtype, "hsn_csr_messages_bwd");
    HSN_REQUIRE(deterministic == 0 || deterministic == 1, HSN_ERR_INVALID_ARGUMENT,
                "hsn_csr_messages_bwd: deterministic must be 0 or 1");
    HSN_REQUIRE(h && indptr && V && cell_idx && grad_m && grad_h && grad_V &&
                    (E == 0 || (indices && a && grad_a)),
                HSN_ERR_INVALID_ARGUMENT, "hsn_csr_messages_bwd: a pointer is NULL");
    by_dtype<RunCsrBwd>(dtype, h, indptr, indices, a, V, cell_idx, grad_m, grad_h, grad_a, grad_V,
                        B, N, d, K, E, as_stream(stream));
    HSN_HIP(hipGetLastError());
    HSN_ABI_END
}
