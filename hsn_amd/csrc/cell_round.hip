// The fused cell round of one position on gfx950 (reference kernels/cuda/hsn_window.cu:226-531,
// hsn_win_cell_front / _routes / _mlp_hidden / _mlp_out / _cell_back; contract: PDGCell.step_sparse
// and the tick, python/hsn/model/cell.py:349-505 and python/hsn/model/state.py:316-324).
//
// Two launches a position, fp32 throughout, every product on v_mfma_f32_16x16x4_f32 tiles:
//   units  (row tile, hidden chunk) workgroups: the row tiles of every unit's valid slots (16
//          slots of one unit in slot order, laid end to end unit after unit, as many as the slots
//          need: no separate routing launch) times the chunks of 64 hidden units. A workgroup
//          finds its unit and slots, puts the unit's first-layer weights in flight, and meanwhile
//          builds its slots' inputs itself: each slot's weighted source sum, m = V (sum), the 4d
//          input [u; eps; h_i; m] and the cell norm. Then hidden = v W1_j + b1_j (the four
//          wavefronts split the reduction and sum their shares in a fixed order), the GELU, and
//          the chunk's share of F = act W2_j, stored per chunk and summed in chunk order by the
//          next launch (no atomics). The gate's 16-column tiles go to the chunks (tile c to the
//          chunk-c workgroup, its wavefronts splitting the reduction; chunk 0 takes every tile
//          when there are fewer chunks than tiles).
//   back   (row, part) workgroups: part 0 finishes F (+ b2_j), W_out, the candidate norm, tanh and
//          the gated update of the row's slots, then q and h_sel; parts 1.. copy the row's other
//          cells, 64 a workgroup, and tick the ages. Written cells and copied cells are disjoint,
//          so the parts need no ordering between them.
// Latency, not bandwidth or arithmetic, bounds a position at the model's sizes (a few MB of
// weights and state, a few MFLOP): every global load is issued as early as what it depends on
// allows, in batches, and products read their LDS operands a block ahead of the MFMAs.
#include <climits>
#include <string>

#include "../../include/hsn_ops.h"
#include "../../include/hsn_round.h"
#include "abi_util.h"
#include "common.cuh"
#include "dpp.cuh"

namespace hsn {
// Raise a kernel's dynamic-LDS limit to 160 KiB once per (kernel, device) (runtime.cpp).
hipError_t allow_lds_raw(const void* kernel, size_t lds);

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kRoundThreads = 256;
constexpr int kRoundWaves = kRoundThreads / kWave;
constexpr int kRows = 16;         // slots a row tile (the MFMA tile's rows)
constexpr int kChunk = 16 * kRoundWaves;  // hidden units a chunk: a 16-column tile a wavefront
constexpr int kCopyCells = 64;    // cells a copy workgroup of the back launch
constexpr int kMaxSlots = 8192;   // B K: the units launch caches every slot's unit and cell
constexpr int kMaxUnits = 255;    // units fit a byte, 0xff marks a padded slot
constexpr int kMaxD = 256;
constexpr int kDefaultLds = 64 * 1024;
constexpr int kMaxLds = 160 * 1024;

__host__ __device__ inline int64_t align_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
__host__ __device__ inline int chunks_of(int H) { return (H + kChunk - 1) / kChunk; }

// The scratch: the gate [P, d], F's chunk shares [chunks, P, d] (P = B K).
struct Work {
    int64_t gate, part, bytes;
};
__host__ __device__ inline Work work_of(int B, int K, int d, int H) {
    const int64_t P = int64_t(B) * K;
    Work w;
    w.gate = 0;
    w.part = align_up(w.gate + 4 * P * d, 256);
    w.bytes = align_up(w.part + 4 * int64_t(chunks_of(H)) * P * d, 256);
    return w;
}

// LDS of each launch (rows padded by one float: the 16 rows of a tile fall on distinct banks).
struct UnitsLds {
    int ucache, ccache, count, rows, meta, cell, src, w, gain, b1, gb, hbar, x, red, gred, act, sh, sx,
        sr, sa, bytes;
};
__host__ __device__ inline UnitsLds units_lds(int P, int d, int D) {
    UnitsLds L;
    L.sh = d + 1;
    L.sx = 4 * d + 1;
    L.sr = kChunk + 1;
    L.sa = kChunk + 1;
    L.ucache = 0;                                    // uint8 [P]: each slot's unit, 0xff padded
    L.ccache = static_cast<int>(align_up(P, 16));    // int [P]: each slot's cell
    L.count = L.ccache + 4 * P;                      // int [256]: the valid slots of each unit
    L.rows = L.count + 4 * 256;                      // int [16]: the tile's slots, -1 past the end
    L.meta = L.rows + 4 * kRows;                     // int [4]
    L.cell = L.meta + 16;                            // int [16]: the tile's cells
    L.src = L.cell + 4 * kRows;                      // int [16][D]: their sources, -1 absent
    L.w = L.src + 4 * kRows * D;                     // float [16][D]: their edge weights
    L.gain = L.w + 4 * kRows * D;                    // float [4 d]: the cell norm's gain
    L.b1 = L.gain + 4 * 4 * d;                       // float [64]: the chunk's first-layer bias
    L.gb = L.b1 + 4 * kChunk;                        // float [16]: the gate tile's bias
    L.hbar = L.gb + 4 * 16;                          // float [16][sh]: the weighted source sums
    L.x = L.hbar + 4 * kRows * L.sh;                 // float [16][sx]: the inputs, then v
    L.red = L.x + 4 * kRows * L.sx;                  // float [4][16][sr]: the waves' hidden shares
    L.gred = L.red + 4 * kRoundWaves * kRows * L.sr;  // float [4][16][17]: the gate tile's shares
    L.act = L.gred + 4 * kRoundWaves * kRows * 17;   // float [16][sa]
    L.bytes = L.act + 4 * kRows * L.sa;
    return L;
}
struct BackLds {
    int cell, unit, flag, alpha, qrow, cgain, o, pre, old, gate, scale, so, k16, bytes;
};
__host__ __device__ inline BackLds back_lds(int K, int d) {
    BackLds L;
    L.k16 = (K + 15) / 16 * 16;
    L.so = d + 1;
    L.cell = 0;                          // int [k16]
    L.unit = L.cell + 4 * L.k16;         // int [k16]
    L.flag = L.unit + 4 * L.k16;         // int [64]: the copy part's written cells
    L.alpha = L.flag + 4 * kCopyCells;   // float [k16]: the slots' alpha
    L.qrow = L.alpha + 4 * L.k16;        // float [d]: the row's summary
    L.cgain = L.qrow + 4 * d;            // float [d]: the candidate norm's gain
    L.o = L.cgain + 4 * d;               // float [k16][so]: F (mixed), then the new states
    L.pre = L.o + 4 * L.k16 * L.so;      // float [k16][so]: W_out's output, then the changes
    L.old = L.pre + 4 * L.k16 * L.so;    // float [k16][so]: the slots' states before the round
    L.gate = L.old + 4 * L.k16 * L.so;   // float [k16][so]: their gates
    L.scale = L.gate + 4 * L.k16 * L.so; // float [k16]
    L.bytes = L.scale + 4 * L.k16;
    return L;
}

// A slot's cell when it is written (valid, cell in [0, N)), else -1.
__device__ __forceinline__ int live_cell(const hsn_cell_round& s, int64_t p) {
    const uint8_t ok = s.valid[p];  // both loads issued together
    const int64_t c = s.cells[p];
    return ok && c >= 0 && c < s.N ? static_cast<int>(c) : -1;
}
__device__ __forceinline__ int unit_of(const hsn_cell_round& s, int64_t p) {
    const int64_t j = s.units[p];
    return static_cast<int>(j < 0 ? 0 : (j >= s.M ? s.M - 1 : j));
}

__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// One 16 x 16 tile of A (16 rows in LDS, this lane's row at `a`) times B (kdim x 16), kdim =
// 4 q. Lane l supplies A[l % 16][k] and B[k][l % 16] for one k of each 4-step
// (v_mfma_f32_16x16x4_f32's layout): here lane group g = l / 16 walks the quarter
// [g q, (g + 1) q) in order, which sums the same terms with A's row and, for row-major weights,
// B's row read contiguously. `a` and `load(s)` give the lane's A and B at step s of its quarter;
// the first PRE steps' B come from `pre` (registers loaded early, when `use_pre`), the rest are
// loaded 16 steps at a time, a block ahead of the products. Returns D[4 g + r][l % 16] in element
// r. Every lane of the wavefront calls it (MFMA runs on the whole wavefront); q is uniform.
constexpr int kBlock = 16;

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int PRE, typename Load>
__device__ __forceinline__ v4f product(const float* a, int q, const float (&pre)[PRE],
                                       bool use_pre, Load load) {
    auto rd = [&](int i) { return a[i]; };
    v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    int s = 0;
    if (use_pre && q >= PRE) {  // A read 16 steps at a time: the reads overlap, not the products
#pragma unroll
        for (int b0 = 0; b0 < PRE; b0 += kBlock) {
            float av[kBlock];
#pragma unroll
            for (int i = 0; i < kBlock; ++i) av[i] = rd(b0 + i);
#pragma unroll
            for (int i = 0; i < kBlock; i += 2) {
                acc0 = mfma(av[i], pre[b0 + i], acc0);
                acc1 = mfma(av[i + 1], pre[b0 + i + 1], acc1);
            }
        }
        s = PRE;
    } else if (use_pre) {  // q < PRE (register arrays take compile-time indices only)
#pragma unroll
        for (int i = 0; i < PRE; ++i)
            if (i < q) acc0 = mfma(rd(i), pre[i], acc0);
        s = q;
    }
    const int blocks = (q - s) / kBlock;
    float cur[kBlock], nxt[kBlock];
    if (blocks > 0) {
#pragma unroll
        for (int i = 0; i < kBlock; ++i) cur[i] = load(s + i);
    }
    for (int bi = 0; bi < blocks; ++bi) {
        const int s0 = s + bi * kBlock;
        if (bi + 1 < blocks) {
#pragma unroll
            for (int i = 0; i < kBlock; ++i) nxt[i] = load(s0 + kBlock + i);
        }
        float av[kBlock];
#pragma unroll
        for (int i = 0; i < kBlock; ++i) av[i] = rd(s0 + i);
#pragma unroll
        for (int i = 0; i < kBlock; i += 2) {
            acc0 = mfma(av[i], cur[i], acc0);
            acc1 = mfma(av[i + 1], cur[i + 1], acc1);
        }
#pragma unroll
        for (int i = 0; i < kBlock; ++i) cur[i] = nxt[i];
    }
    for (int t = s + blocks * kBlock; t < q; ++t) acc0 = mfma(rd(t), load(t), acc0);
    return acc0 + acc1;
}

// A lane's first PRE B values of a row-major weight read along its row (w: the lane's row at its
// quarter's start, q steps): 16-byte loads where the row allows them.
template <int PRE>
__device__ __forceinline__ void preload_row(float (&pre)[PRE], const float* w, int q, bool ok) {
    if ((q & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
#pragma unroll
        for (int i = 0; i < PRE; i += 4) {
            float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (ok && i < q) t = *reinterpret_cast<const float4*>(w + i);
            pre[i] = t.x;
            pre[i + 1] = t.y;
            pre[i + 2] = t.z;
            pre[i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < PRE; ++i) pre[i] = ok && i < q ? w[i] : 0.0f;
    }
}

// A lane's first PRE B values of a weight read down its column (w: the lane's column at its
// quarter's first row, rows `ld` apart, q steps, the rows at or past `rows` reading 0).
template <int PRE>
__device__ __forceinline__ void preload_col(float (&pre)[PRE], const float* w, int64_t ld, int q,
                                            int rows, bool ok) {
#pragma unroll
    for (int i = 0; i < PRE; ++i) pre[i] = ok && i < q && i < rows ? w[i * ld] : 0.0f;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// ---- units: the slots' inputs and their unit's MLP, 64 hidden units a workgroup -----------------
constexpr int kPreGate = 16;  // gate weights a lane holds early (its share of one gate tile)
constexpr int kPreV = 16;     // V weights likewise
constexpr int kPreW1 = 16;    // first-layer steps (float4: four column tiles) a lane holds early
constexpr int kPreW2 = 16;    // second-layer weights (all of a chunk's)

// Four consecutive weights of a row from column `c` on, 0 past `cols` (16-byte loads where the
// row allows them).
__device__ __forceinline__ float4 row4(const float* w, int c, int cols, bool aligned) {
    if (aligned && c + 4 <= cols) return ld4(w + c);
    float4 t;
    t.x = c < cols ? w[c] : 0.0f;
    t.y = c + 1 < cols ? w[c + 1] : 0.0f;
    t.z = c + 2 < cols ? w[c + 2] : 0.0f;
    t.w = c + 3 < cols ? w[c + 3] : 0.0f;
    return t;
}

__global__ __launch_bounds__(kRoundThreads) void round_units(hsn_cell_round s) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int d = s.d, n = 4 * d, M = s.M, H = s.H, N = s.N, D = s.D, K = s.K;
    const int P = s.B * K;
    const UnitsLds L = units_lds(P, d, D);
    uint8_t* ucache = lds + L.ucache;
    int* ccache = reinterpret_cast<int*>(lds + L.ccache);
    int* count = reinterpret_cast<int*>(lds + L.count);
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    int* cell_of = reinterpret_cast<int*>(lds + L.cell);
    int* srcs = reinterpret_cast<int*>(lds + L.src);
    float* ws = reinterpret_cast<float*>(lds + L.w);
    float* gain = reinterpret_cast<float*>(lds + L.gain);
    float* b1c = reinterpret_cast<float*>(lds + L.b1);
    float* hbar = reinterpret_cast<float*>(lds + L.hbar);
    float* x = reinterpret_cast<float*>(lds + L.x);
    float* red = reinterpret_cast<float*>(lds + L.red);
    float* act = reinterpret_cast<float*>(lds + L.act);
    float* gred = reinterpret_cast<float*>(lds + L.gred);
    float* gb = reinterpret_cast<float*>(lds + L.gb);
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int lr = lane & 15, g = lane >> 4;
    const int chunk = blockIdx.y;
    const int h0 = chunk * kChunk;
    const bool lead = chunk == 0;
    const int tiles_d = (d + 15) / 16;
    const Work W = work_of(s.B, K, d, H);
    float* gate_out = reinterpret_cast<float*>(static_cast<unsigned char*>(s.work) + W.gate);
    float* part = reinterpret_cast<float*>(static_cast<unsigned char*>(s.work) + W.part);

    // ---- the position's units and cells; which unit's which row tile this workgroup takes ----
    for (int j = tid; j < M; j += kRoundThreads) count[j] = 0;
    // the first slots' decisions and the norm's gain
    const bool q_first = tid < P;
    const uint8_t valid0 = q_first ? s.valid[tid] : uint8_t(0);
    const int64_t cell0 = q_first ? s.cells[tid] : int64_t(-1);
    const int64_t unit0 = q_first ? s.units[tid] : int64_t(0);
    const float gain0 = tid < n ? s.norm_w[tid] : 0.0f;
    if (q_first) {
        const bool live = valid0 && cell0 >= 0 && cell0 < N;
        const int unit = static_cast<int>(unit0 < 0 ? 0 : (unit0 >= M ? M - 1 : unit0));
        ucache[tid] = live ? static_cast<uint8_t>(unit) : uint8_t(0xff);
        ccache[tid] = live ? static_cast<int>(cell0) : -1;
    }
    for (int q = tid + kRoundThreads; q < P; q += kRoundThreads) {
        const int cell = live_cell(s, q);
        ucache[q] = cell >= 0 ? static_cast<uint8_t>(unit_of(s, q)) : uint8_t(0xff);
        ccache[q] = cell;
    }
    if (tid < n) gain[tid] = gain0;
    for (int c = tid + kRoundThreads; c < n; c += kRoundThreads) gain[c] = s.norm_w[c];
    __syncthreads();
    // the slot-independent weights of the products before the MLP, in flight from here on. The
    // gate's column tiles go to the chunks (tile c to chunk c, the four wavefronts splitting its
    // reduction) when there are as many chunks as tiles; otherwise chunk 0 computes them all.
    const bool split_gate = static_cast<int>(gridDim.y) >= tiles_d;
    const int gtile = split_gate && chunk < tiles_d ? chunk : -1;
    const int qg = n / 16;                      // a lane group's steps of the split gate tile
    const int kg = wave * (n / 4) + g * qg;     // their first reduction index
    const int gcol = gtile * 16 + lr;
    const bool okg = gtile >= 0 && gcol < d;
    const float* gw = s.gate_w + int64_t(okg ? gcol : 0) * n + kg;
    float gpre[kPreGate], vpre[kPreV];
    preload_row(gpre, gw, qg, okg);
    const int colv = wave * 16 + lr;
    preload_row(vpre, s.V + int64_t(wave < tiles_d && colv < d ? colv : 0) * d + g * (d / 4),
                d / 4, wave < tiles_d && colv < d);
    const float gbias0 = gtile >= 0 && tid < 16 && gtile * 16 + tid < d ? s.gate_b[gtile * 16 + tid]
                                                                     : 0.0f;
    for (int q = tid; q < P; q += kRoundThreads)  // integer counts: any order gives the same
        if (ucache[q] != 0xff) atomicAdd(&count[ucache[q]], 1);
    __syncthreads();
    if (wave == 0) {
        int unit = -1, tile = 0;
        if (lane == 0) {
            int before = 0;
            for (int j = 0; j < M; ++j) {
                const int tiles = (count[j] + kRows - 1) / kRows;
                if (static_cast<int>(blockIdx.x) < before + tiles) {
                    unit = j;
                    tile = blockIdx.x - before;
                    break;
                }
                before += tiles;
            }
        }
        unit = readlane(unit, 0);
        tile = readlane(tile, 0);
        if (lane < kRows) {
            rows[lane] = -1;
            cell_of[lane] = -1;
        }
        if (unit >= 0) {
            const int first = tile * kRows;
            int base = 0;
            for (int q0 = 0; q0 < P && base < first + kRows; q0 += kWave) {
                const int q = q0 + lane;
                const bool mine = q < P && ucache[q] == unit;
                const uint64_t m = ballot(mine);
                const int rank = base + lanes_below(m);
                if (mine && rank >= first && rank < first + kRows) {
                    rows[rank - first] = q;
                    cell_of[rank - first] = ccache[q];
                }
                base += __popcll(m);
            }
        }
        if (lane == 0) meta[0] = unit;
    }
    __syncthreads();
    const int j = meta[0];
    if (j < 0) return;  // past the last row tile (uniform)

    // ---- the tile's in-edges, then the unit's weights in flight while the inputs come in ----
    const bool e_first = tid < kRows * D;
    const int ecell0 = e_first ? cell_of[tid / D] : -1;
    const int64_t esrc0 = ecell0 >= 0 ? s.pad_src[int64_t(ecell0) * D + tid % D] : int64_t(-1);
    const float ew0 = ecell0 >= 0 ? s.edge_w[int64_t(ecell0) * D + tid % D] : 0.0f;
    // first layer: wavefront w takes the reduction quarter [w n / 4, (w + 1) n / 4) of all 64
    // columns, lane group g its q1 = n / 16 steps from k = w n / 4 + g q1; a 16-byte load gives
    // four column tiles (tile t's column i is h0 + 4 i + t)
    const int q1 = n / 16;
    const int k1 = wave * (n / 4) + g * q1;
    const int c1 = h0 + 4 * lr;
    const float* w1 = s.W1 + (int64_t(j) * n + k1) * H;
    const bool al1 = (H & 3) == 0;
    float4 w1pre[kPreW1];
#pragma unroll
    for (int i = 0; i < kPreW1; ++i)
        w1pre[i] = i < q1 ? row4(w1 + int64_t(i) * H, c1, H, al1) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float bias1 = tid < kChunk && h0 + tid < H ? s.b1[int64_t(j) * H + h0 + tid] : 0.0f;
    // second layer: as before, a 16-column tile a wavefront over the chunk's 64 rows
    const int col2 = wave * 16 + lr;
    const bool ok2 = wave < tiles_d && col2 < d;
    const int rows2 = H - h0 - g * (kChunk / 4);  // the chunk's rows left from this lane's quarter
    const float* w2 = s.W2 + (int64_t(j) * H + h0 + g * (kChunk / 4)) * d + (ok2 ? col2 : 0);
    float w2pre[kPreW2];
    preload_col(w2pre, w2, d, kChunk / 4, rows2, ok2);
    if (e_first) {
        srcs[tid] = esrc0 >= 0 && esrc0 < N ? static_cast<int>(esrc0) : -1;
        ws[tid] = ew0;
    }
    for (int e = tid + kRoundThreads; e < kRows * D; e += kRoundThreads) {
        const int cell = cell_of[e / D];
        int64_t src = -1;
        float w = 0.0f;
        if (cell >= 0) {
            src = s.pad_src[int64_t(cell) * D + e % D];
            w = s.edge_w[int64_t(cell) * D + e % D];
        }
        srcs[e] = src >= 0 && src < N ? static_cast<int>(src) : -1;
        ws[e] = w;
    }
    if (tid < kChunk) b1c[tid] = bias1;
    if (tid < 16) gb[tid] = gbias0;
    __syncthreads();

    // ---- the inputs: the state blocks and each slot's weighted source sum, four columns a thread
    const int d4 = d / 4;
    for (int e = tid; e < kRows * d4; e += kRoundThreads) {
        const int pp = e / d4, c = 4 * (e % d4);
        const int cell = cell_of[pp];
        float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f), uu = sum, ee = sum, hh = sum;
        if (cell >= 0) {
            const int64_t r = rows[pp] / K;
            const float* hr = s.h + r * N * d;
            uu = ld4(s.u + r * d + c);
            ee = ld4(s.eps + r * d + c);
            hh = ld4(hr + int64_t(cell) * d + c);
#pragma unroll 8
            for (int k = 0; k < D; ++k) {
                const int src = srcs[pp * D + k];
                const float w = ws[pp * D + k];
                const float4 hv = src >= 0 ? ld4(hr + int64_t(src) * d + c)
                                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                sum.x += w * hv.x;
                sum.y += w * hv.y;
                sum.z += w * hv.z;
                sum.w += w * hv.w;
            }
        }
        float* hb = hbar + pp * L.sh + c;
        float* xr = x + pp * L.sx + c;
        hb[0] = sum.x, hb[1] = sum.y, hb[2] = sum.z, hb[3] = sum.w;
        xr[0] = uu.x, xr[1] = uu.y, xr[2] = uu.z, xr[3] = uu.w;
        xr[d] = ee.x, xr[d + 1] = ee.y, xr[d + 2] = ee.z, xr[d + 3] = ee.w;
        xr[2 * d] = hh.x, xr[2 * d + 1] = hh.y, xr[2 * d + 2] = hh.z, xr[2 * d + 3] = hh.w;
    }
    __syncthreads();

    // m = V hbar: B[k][col] = V[col][k]
    for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
        const int col = tile * 16 + lr;
        const bool ok = col < d;
        const float* vrow = s.V + int64_t(ok ? col : 0) * d + g * (d / 4);
        const v4f acc = product(hbar + lr * L.sh + g * (d / 4), d / 4, vpre, tile == wave,
                                [&](int k) {
                                    const float w = vrow[k];
                                    return ok ? w : 0.0f;
                                });
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (ok) x[(4 * g + r) * L.sx + 3 * d + col] = acc[r];
    }
    __syncthreads();

    // the cell norm: 1 / sqrt(mean(x^2) + eps) a slot, a wavefront four slots side by side, then
    // v = x scale gain in place (the wavefront's own rows; one read of each value when a row is
    // at most four values a lane)
    {
        constexpr int kPer = kRows / kRoundWaves;
        float ss[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) ss[i] = 0.0f;
        const bool one_pass = n <= 4 * kWave;
        float t[kPer][4];
        if (one_pass) {
#pragma unroll
            for (int i = 0; i < kPer; ++i)
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int c = lane + m * kWave;
                    t[i][m] = c < n ? x[(wave * kPer + i) * L.sx + c] : 0.0f;
                    ss[i] += t[i][m] * t[i][m];
                }
        } else {
            for (int c = lane; c < n; c += kWave) {
#pragma unroll
                for (int i = 0; i < kPer; ++i) {
                    const float v = x[(wave * kPer + i) * L.sx + c];
                    ss[i] += v * v;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) ss[i] = group_sum<kWave>(ss[i]);
        float scale[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) scale[i] = rsqrtf(ss[i] / static_cast<float>(n) + s.norm_eps);
        if (one_pass) {
#pragma unroll
            for (int i = 0; i < kPer; ++i)
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int c = lane + m * kWave;
                    if (c < n) x[(wave * kPer + i) * L.sx + c] = t[i][m] * scale[i] * gain[c];
                }
        } else {
            for (int c = lane; c < n; c += kWave) {
#pragma unroll
                for (int i = 0; i < kPer; ++i)
                    x[(wave * kPer + i) * L.sx + c] = x[(wave * kPer + i) * L.sx + c] * scale[i] *
                                                      gain[c];
            }
        }
    }
    __syncthreads();

    // the gate: sigmoid(gate_w v + gate_b), B[k][col] = gate_w[col][k]
    if (gtile >= 0) {  // this wavefront's share of the chunk's tile, summed after the hidden layer
        const v4f acc = product(x + lr * L.sx + kg, qg, gpre, true, [&](int k) {
            const float w = gw[k];
            return okg ? w : 0.0f;
        });
#pragma unroll
        for (int r = 0; r < 4; ++r) gred[(wave * kRows + 4 * g + r) * 17 + lr] = acc[r];
    } else if (!split_gate && lead) {  // fewer chunks than tiles: chunk 0 takes them all
        const float none[kBlock] = {};
        for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
            const int col = tile * 16 + lr;
            const bool ok = col < d;
            const float* grow = s.gate_w + int64_t(ok ? col : 0) * n + g * d;
            const v4f acc = product(x + lr * L.sx + g * d, d, none, false, [&](int k) {
                const float w = grow[k];
                return ok ? w : 0.0f;
            });
            const float bias = ok ? s.gate_b[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = rows[4 * g + r];
                if (ok && q >= 0) gate_out[int64_t(q) * d + col] = act_sigmoid(acc[r] + bias);
            }
        }
    }

    // hidden = v W1_j + b1_j: each wavefront its quarter of the reduction for four column tiles
    {
        v4f acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        const float* arow = x + lr * L.sx + k1;
        auto steps = [&](const float4* b, int s0, int cnt) {
            // cnt is kBlock or less; the A reads go first
            float av[kBlock];
#pragma unroll
            for (int i = 0; i < kBlock; ++i) av[i] = i < cnt ? arow[s0 + i] : 0.0f;
#pragma unroll
            for (int i = 0; i < kBlock; ++i) {
                if (i < cnt) {
                    acc[0] = mfma(av[i], b[i].x, acc[0]);
                    acc[1] = mfma(av[i], b[i].y, acc[1]);
                    acc[2] = mfma(av[i], b[i].z, acc[2]);
                    acc[3] = mfma(av[i], b[i].w, acc[3]);
                }
            }
        };
        steps(w1pre, 0, q1 < kPreW1 ? q1 : kPreW1);
        for (int s0 = kPreW1; s0 < q1; s0 += kBlock) {
            float4 b[kBlock];
#pragma unroll
            for (int i = 0; i < kBlock; ++i)
                b[i] = s0 + i < q1 ? row4(w1 + int64_t(s0 + i) * H, c1, H, al1)
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            steps(b, s0, q1 - s0 < kBlock ? q1 - s0 : kBlock);
        }
        // the wavefront's share: row 4 g + r, column 4 lr + t of the chunk
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[(wave * kRows + 4 * g + r) * L.sr + 4 * lr + t] = acc[t][r];
    }
    __syncthreads();
    for (int e = tid; e < kRows * kChunk; e += kRoundThreads) {  // the shares in wave order
        const int row = e / kChunk, c = e % kChunk;
        float z = 0.0f;
#pragma unroll
        for (int w = 0; w < kRoundWaves; ++w) z += red[(w * kRows + row) * L.sr + c];
        act[row * L.sa + c] = h0 + c < H ? gelu_erf(z + b1c[c]) : 0.0f;
    }
    if (gtile >= 0 && tid < kRows * 16) {  // the gate tile's shares in wave order
        const int row = tid / 16, c = tid % 16;
        const int col = gtile * 16 + c, q = rows[row];
        float z = 0.0f;
#pragma unroll
        for (int w = 0; w < kRoundWaves; ++w) z += gred[(w * kRows + row) * 17 + c];
        if (col < d && q >= 0) gate_out[int64_t(q) * d + col] = act_sigmoid(z + gb[c]);
    }
    __syncthreads();

    // this chunk's share of F = act W2_j: B[k][col] = W2[j][h0 + k][col]
    for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
        const int col = tile * 16 + lr;
        const bool ok = col < d;
        const float* w2t = s.W2 + (int64_t(j) * H + h0 + g * (kChunk / 4)) * d + (ok ? col : 0);
        const v4f acc = product(act + lr * L.sa + g * (kChunk / 4), kChunk / 4, w2pre,
                                tile == wave, [&](int k) {
                                    const int kk = k < rows2 ? k : 0;  // past H: row 0, unused
                                    const float w = w2t[int64_t(kk) * d];
                                    return ok && k < rows2 ? w : 0.0f;
                                });
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = rows[4 * g + r];
            if (ok && q >= 0) part[(int64_t(chunk) * P + q) * d + col] = acc[r];
        }
    }
}

// ---- back: W_out, candidate, update, q, h_sel; the other cells' copy and the tick --------------
constexpr int kPreWout = 16;  // W_out weights a lane loads before anything else (all at d 64)

__global__ __launch_bounds__(kRoundThreads) void round_back(hsn_cell_round s) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int d = s.d, K = s.K, N = s.N;
    const int64_t P = int64_t(s.B) * K;
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const BackLds L = back_lds(K, d);
    int* kcell = reinterpret_cast<int*>(lds + L.cell);
    int* kunit = reinterpret_cast<int*>(lds + L.unit);
    const float* h = s.h + r * N * d;
    float* h_new = s.h_new + r * N * d;

    for (int k = tid; k < L.k16; k += kRoundThreads) {
        kcell[k] = k < K ? live_cell(s, r * K + k) : -1;
        kunit[k] = k < K ? unit_of(s, r * K + k) : 0;
        if (blockIdx.y == 0) reinterpret_cast<float*>(lds + L.alpha)[k] = k < K ? s.alpha[r * K + k] : 0.0f;
    }
    if (blockIdx.y == 0) {  // the row's summary and the candidate norm's gain
        for (int c = tid; c < d; c += kRoundThreads) {
            reinterpret_cast<float*>(lds + L.qrow)[c] = s.q[r * d + c];
            reinterpret_cast<float*>(lds + L.cgain)[c] = s.cand_norm ? s.cand_w[c] : 0.0f;
        }
    }
    // the wavefront's first W_out tile, in flight meanwhile (the slot part's only)
    const int tiles_d = (d + 15) / 16;
    const int lr = lane & 15, g = lane >> 4;
    const bool lead = blockIdx.y == 0;
    const int col0 = (wave % tiles_d) * 16 + lr;
    const bool ok0 = lead && wave < (L.k16 / 16) * tiles_d && col0 < d;
    float wpre[kPreWout];
    preload_row(wpre, s.W_out + int64_t(ok0 ? col0 : 0) * d + g * (d / 4), d / 4, ok0);
    __syncthreads();

    if (blockIdx.y > 0) {  // copy cells c0 .. c0 + 63 except the written ones, tick their ages
        const int c0 = (blockIdx.y - 1) * kCopyCells;
        int* written = reinterpret_cast<int*>(lds + L.flag);
        for (int i = tid; i < kCopyCells; i += kRoundThreads) written[i] = 0;
        __syncthreads();
        for (int k = tid; k < K; k += kRoundThreads) {
            const int c = kcell[k];
            if (c >= c0 && c < c0 + kCopyCells) written[c - c0] = 1;
        }
        __syncthreads();
        const int cells = min(kCopyCells, N - c0);
        const int d4 = d / 4;
        const float4* src = reinterpret_cast<const float4*>(h + int64_t(c0) * d);
        float4* dst = reinterpret_cast<float4*>(h_new + int64_t(c0) * d);
        for (int e = tid; e < cells * d4; e += kRoundThreads)
            if (!written[e / d4]) dst[e] = src[e];
        for (int i = tid; i < cells; i += kRoundThreads) {
            const int64_t at = r * N + c0 + i;
            s.age_new[at] = written[i] ? 0 : s.age[at] + 1;
        }
        return;
    }

    float* o = reinterpret_cast<float*>(lds + L.o);
    float* pre = reinterpret_cast<float*>(lds + L.pre);
    float* scale = reinterpret_cast<float*>(lds + L.scale);
    float* olds = reinterpret_cast<float*>(lds + L.old);
    float* gates = reinterpret_cast<float*>(lds + L.gate);
    const float* alphas = reinterpret_cast<const float*>(lds + L.alpha);
    const float* qrow = reinterpret_cast<const float*>(lds + L.qrow);
    const float* cgain = reinterpret_cast<const float*>(lds + L.cgain);
    const Work W = work_of(s.B, K, d, s.H);
    const float* gate = reinterpret_cast<const float*>(static_cast<unsigned char*>(s.work) + W.gate);
    const float* part = reinterpret_cast<const float*>(static_cast<unsigned char*>(s.work) + W.part);
    const int chunks = chunks_of(s.H);

    // F = the chunks' shares in chunk order + b2_j (alpha before W_out without the candidate
    // norm), four columns a thread; the slots' old states and gates come into LDS in the same
    // round trip
    const int d4 = d / 4;
    for (int e = tid; e < L.k16 * d4; e += kRoundThreads) {
        const int k = e / d4, xc = 4 * (e % d4);
        const int cell = kcell[k];
        float4 val = make_float4(0.0f, 0.0f, 0.0f, 0.0f), old = val, b = val;
        if (cell >= 0) {
            const int64_t p = r * K + k;
            float4 f = val;
#pragma unroll 8
            for (int c = 0; c < chunks; ++c) {
                const float4 t = ld4(part + (int64_t(c) * P + p) * d + xc);
                f.x += t.x, f.y += t.y, f.z += t.z, f.w += t.w;
            }
            const float4 bias = ld4(s.b2 + int64_t(kunit[k]) * d + xc);
            old = ld4(h + int64_t(cell) * d + xc);
            b = ld4(gate + p * d + xc);
            f.x += bias.x, f.y += bias.y, f.z += bias.z, f.w += bias.w;
            const float a = s.cand_norm ? 1.0f : alphas[k];
            val = s.cand_norm ? f : make_float4(a * f.x, a * f.y, a * f.z, a * f.w);
        }
        float* orow = o + k * L.so + xc;
        float* hrow = olds + k * L.so + xc;
        float* grow = gates + k * L.so + xc;
        orow[0] = val.x, orow[1] = val.y, orow[2] = val.z, orow[3] = val.w;
        hrow[0] = old.x, hrow[1] = old.y, hrow[2] = old.z, hrow[3] = old.w;
        grow[0] = b.x, grow[1] = b.y, grow[2] = b.z, grow[3] = b.w;
    }
    __syncthreads();

    // pre = W_out o: B[k][col] = W_out[col][k], tiles over (slot tile, column tile)
    for (int tile = wave; tile < (L.k16 / 16) * tiles_d; tile += kRoundWaves) {
        const int rt = tile / tiles_d, ct = tile % tiles_d;
        const int col = ct * 16 + lr;
        const bool ok = col < d;
        const float* wrow = s.W_out + int64_t(ok ? col : 0) * d + g * (d / 4);
        const v4f acc = product(o + (rt * 16 + lr) * L.so + g * (d / 4), d / 4, wpre,
                                tile == wave, [&](int k) {
                                    const float w = wrow[k];
                                    return ok ? w : 0.0f;
                                });
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (ok) pre[(rt * 16 + 4 * g + i) * L.so + col] = acc[i];
    }
    __syncthreads();

    if (s.cand_norm) {  // 1 / sqrt(mean(y^2) + eps) a slot, a wavefront a slot
        for (int k = wave; k < K; k += kRoundWaves) {
            float ss = 0.0f;
            for (int c = lane; c < d; c += kWave) {
                const float t = pre[k * L.so + c];
                ss += t * t;
            }
            ss = group_sum<kWave>(ss);
            if (lane == 0) scale[k] = rsqrtf(ss / static_cast<float>(d) + s.cand_eps);
        }
        __syncthreads();
    }

    // c = tanh(...), the gated update of the written cells; o takes the new state, pre the change
    for (int e = tid; e < K * d; e += kRoundThreads) {
        const int k = e / d, xc = e % d;
        const int cell = kcell[k];
        float next = 0.0f, change = 0.0f;
        if (cell >= 0) {
            const float y = pre[k * L.so + xc];
            const float value = s.cand_norm ? alphas[k] * (y * scale[k] * cgain[xc]) : y;
            const float c = tanhf(value);
            const float old = olds[k * L.so + xc];
            const float b = gates[k * L.so + xc];
            next = (1.0f - b) * old + b * c;
            change = next - old;
            h_new[int64_t(cell) * d + xc] = next;
        }
        o[k * L.so + xc] = next;
        pre[k * L.so + xc] = change;
    }
    __syncthreads();

    // q += the changes' sum (slot order) / N; h_sel: the slot's new state, cell 0's on padding
    for (int xc = tid; xc < d; xc += kRoundThreads) {
        float sum = 0.0f;
        for (int k = 0; k < K; ++k) sum += pre[k * L.so + xc];
        s.q_new[r * d + xc] = qrow[xc] + sum / static_cast<float>(N);
    }
    int zero_slot = -1;  // the slot that wrote cell 0, if any
    for (int k = 0; k < K; ++k)
        if (kcell[k] == 0) zero_slot = k;
    for (int e = tid; e < K * d; e += kRoundThreads) {
        const int k = e / d, xc = e % d;
        float val;
        if (kcell[k] >= 0)
            val = o[k * L.so + xc];
        else
            val = zero_slot >= 0 ? o[zero_slot * L.so + xc] : h[xc];
        s.h_sel[(r * K + k) * d + xc] = val;
    }
}

void round_check(const hsn_cell_round* s) {
    HSN_REQUIRE(s != nullptr, HSN_ERR_INVALID_ARGUMENT, "cell round: NULL descriptor");
    HSN_REQUIRE(s->B >= 1 && s->N >= 1 && s->d >= 1 && s->K >= 1 && s->M >= 1 && s->H >= 1 &&
                    s->D >= 0,
                HSN_ERR_INVALID_ARGUMENT, "cell round: every size must be positive (D >= 0)");
    HSN_REQUIRE(s->d % 4 == 0 && s->d <= kMaxD, HSN_ERR_INVALID_ARGUMENT,
                "cell round: model.d must be a multiple of 4 and at most 256");
    HSN_REQUIRE(s->M <= kMaxUnits, HSN_ERR_INVALID_ARGUMENT, "cell round: more than 255 units");
    HSN_REQUIRE(int64_t(s->B) * s->K <= kMaxSlots, HSN_ERR_INVALID_ARGUMENT,
                "cell round: more than 8192 slots (B K) a position");
    HSN_REQUIRE(s->D <= 1024 && units_lds(s->B * s->K, s->d, s->D).bytes <= kMaxLds,
                HSN_ERR_INVALID_ARGUMENT,
                "cell round: the position's slot table and 16 slots' inputs exceed 160 KiB of LDS");
    HSN_REQUIRE(back_lds(s->K, s->d).bytes <= kMaxLds, HSN_ERR_INVALID_ARGUMENT,
                "cell round: a row's slots (16 K d bytes) exceed 160 KiB of LDS");
    const int64_t P = int64_t(s->B) * s->K;
    HSN_REQUIRE(check_elems({int64_t(s->B) * s->N * s->d, P * s->d,
                             int64_t(chunks_of(s->H)) * P * s->d, int64_t(s->M) * 4 * s->d * s->H,
                             int64_t(s->N) * s->D}),
                HSN_ERR_SIZE_OVERFLOW, "cell round: a buffer is too large");
    const void* need[] = {s->u, s->eps, s->h, s->q, s->age, s->cells, s->units, s->valid,
                          s->alpha, s->V, s->norm_w, s->gate_w, s->gate_b, s->W1, s->b1, s->W2,
                          s->b2, s->W_out, s->work, s->h_new, s->q_new, s->age_new, s->h_sel};
    for (const void* p : need)
        HSN_REQUIRE(p != nullptr, HSN_ERR_INVALID_ARGUMENT, "cell round: a buffer is NULL");
    HSN_REQUIRE(s->D == 0 || (s->edge_w != nullptr && s->pad_src != nullptr),
                HSN_ERR_INVALID_ARGUMENT, "cell round: edge_w / pad_src is NULL with edges");
    HSN_REQUIRE(!s->cand_norm || s->cand_w != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "cell round: the candidate norm's gain is NULL");
    for (const void* p : {static_cast<const void*>(s->work), static_cast<const void*>(s->u),
                          static_cast<const void*>(s->eps), static_cast<const void*>(s->h),
                          static_cast<const void*>(s->h_new)})
        HSN_REQUIRE(reinterpret_cast<uintptr_t>(p) % 16 == 0, HSN_ERR_INVALID_ARGUMENT,
                    "cell round: work, u, eps, h and h_new must be 16-byte aligned");
}

template <typename Kernel>
void launch(Kernel kernel, dim3 grid, int lds, hipStream_t stream, const hsn_cell_round& s) {
    if (lds > kDefaultLds) HSN_HIP(allow_lds_raw(reinterpret_cast<const void*>(kernel), lds));
    hipLaunchKernelGGL(kernel, grid, dim3(kRoundThreads), static_cast<size_t>(lds), stream, s);
    HSN_HIP(hipGetLastError());
}

}  // namespace
}  // namespace hsn

using namespace hsn;

extern "C" int hsn_win_cell_round_check(const hsn_cell_round* round) {
    HSN_ABI_BEGIN
    round_check(round);
    HSN_ABI_END
}

extern "C" int hsn_win_cell_round_workspace(const hsn_cell_round* round, int64_t* bytes) {
    HSN_ABI_BEGIN
    HSN_REQUIRE(round != nullptr && bytes != nullptr, HSN_ERR_INVALID_ARGUMENT,
                "cell round: NULL argument");
    HSN_REQUIRE(round->B >= 1 && round->K >= 1 && round->d >= 1 && round->H >= 1,
                HSN_ERR_INVALID_ARGUMENT, "cell round: every size must be positive");
    *bytes = work_of(round->B, round->K, round->d, round->H).bytes;
    HSN_ABI_END
}

extern "C" int hsn_win_cell_round(const hsn_cell_round* round, void* stream) {
    HSN_ABI_BEGIN
    round_check(round);
    const hsn_cell_round s = *round;
    const hipStream_t st = as_stream(stream);
    const int P = s.B * s.K;
    const unsigned tiles = static_cast<unsigned>((P + kRows - 1) / kRows);
    launch(round_units, dim3(tiles + static_cast<unsigned>(s.M), chunks_of(s.H)),
           units_lds(P, s.d, s.D).bytes, st, s);
    launch(round_back, dim3(s.B, 1 + (s.N + kCopyCells - 1) / kCopyCells),
           back_lds(s.K, s.d).bytes, st, s);
    HSN_ABI_END
}
