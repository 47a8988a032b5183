// The fused cell round of one position on gfx950 (reference kernels/cuda/hsn_window.cu:226-531,
// hsn_win_cell_front / _routes / _mlp_hidden / _mlp_out / _cell_back; contract: PDGCell.step_sparse
// and the tick, python/hsn/model/cell.py:349-505 and python/hsn/model/state.py:316-324).
//
// Three launches a position, fp32 throughout, every product on v_mfma_f32_16x16x4_f32 tiles:
//   front  16 slots a workgroup, in slot order: each slot's weighted source sum, m = V (sum), the
//          4d input [u; eps; h_i; m], the cell norm (one DPP reduction a slot) and the gate's
//          product and sigmoid; the normalised input and the gate go to the scratch.
//   units  (row tile, hidden chunk) workgroups: the row tiles of every unit's valid slots (16
//          slots of one unit in slot order, laid end to end unit after unit, as many as the slots
//          need: no separate routing launch) times the chunks of 64 hidden units: hidden =
//          v W1_j + b1_j, the GELU, and the chunk's share of F = act W2_j, stored per chunk and
//          summed in chunk order by the next launch (a fixed order, no atomics).
//   back   (row, part) workgroups: part 0 finishes F (+ b2_j), W_out, the candidate norm, tanh and
//          the gated update of the row's slots, then q and h_sel; parts 1.. copy the row's other
//          cells, 64 a workgroup, and tick the ages. Written cells and copied cells are disjoint,
//          so the parts need no ordering between them.
// Latency, not bandwidth or arithmetic, bounds a position at the model's sizes (a few MB of
// weights and state, a few MFLOP): the launches are short and their loads are issued in batches.
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
constexpr int kMaxSlots = 16384;  // B K: the units launch caches every slot's unit in LDS
constexpr int kMaxUnits = 255;    // units fit a byte, 0xff marks a padded slot
constexpr int kMaxD = 256;
constexpr int kDefaultLds = 64 * 1024;
constexpr int kMaxLds = 160 * 1024;

__host__ __device__ inline int64_t align_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
__host__ __device__ inline int chunks_of(int H) { return (H + kChunk - 1) / kChunk; }

// The scratch: v [P, 4d], the gate [P, d], F's chunk shares [chunks, P, d] (P = B K).
struct Work {
    int64_t v, gate, part, bytes;
};
__host__ __device__ inline Work work_of(int B, int K, int d, int H) {
    const int64_t P = int64_t(B) * K;
    Work w;
    w.v = 0;
    w.gate = align_up(w.v + 4 * P * 4 * d, 256);
    w.part = align_up(w.gate + 4 * P * d, 256);
    w.bytes = align_up(w.part + 4 * int64_t(chunks_of(H)) * P * d, 256);
    return w;
}

// LDS of each launch (rows padded by one float: the 16 rows of a tile fall on distinct banks).
struct FrontLds {
    int cell, hbar, x, rms, sh, sx, bytes;
};
__host__ __device__ inline FrontLds front_lds(int d) {
    FrontLds L;
    L.sh = d + 1;
    L.sx = 4 * d + 1;
    L.cell = 0;                           // int [16]
    L.hbar = L.cell + 4 * kRows;          // float [16][sh]
    L.x = L.hbar + 4 * kRows * L.sh;      // float [16][sx]
    L.rms = L.x + 4 * kRows * L.sx;       // float [16]
    L.bytes = L.rms + 4 * kRows;
    return L;
}
struct UnitsLds {
    int ucache, rows, meta, v, act, sv, sa, bytes;
};
__host__ __device__ inline UnitsLds units_lds(int P, int d) {
    UnitsLds L;
    L.sv = 4 * d + 1;
    L.sa = kChunk + 1;
    L.ucache = 0;                                    // uint8 [P]
    L.rows = static_cast<int>(align_up(P, 16));      // int [16]
    L.meta = L.rows + 4 * kRows;                     // int [4]
    L.v = L.meta + 16;                               // float [16][sv]
    L.act = L.v + 4 * kRows * L.sv;                  // float [16][sa]
    L.bytes = L.act + 4 * kRows * L.sa;
    return L;
}
struct BackLds {
    int cell, unit, flag, o, pre, scale, so, k16, bytes;
};
__host__ __device__ inline BackLds back_lds(int K, int d) {
    BackLds L;
    L.k16 = (K + 15) / 16 * 16;
    L.so = d + 1;
    L.cell = 0;                          // int [k16]
    L.unit = L.cell + 4 * L.k16;         // int [k16]
    L.flag = L.unit + 4 * L.k16;         // int [64]: the copy part's written cells
    L.o = L.flag + 4 * kCopyCells;       // float [k16][so]: F (mixed), then the new states
    L.pre = L.o + 4 * L.k16 * L.so;      // float [k16][so]: W_out's output, then the changes
    L.scale = L.pre + 4 * L.k16 * L.so;  // float [k16]
    L.bytes = L.scale + 4 * L.k16;
    return L;
}

// A slot's cell when it is written (valid, cell in [0, N)), else -1.
__device__ __forceinline__ int live_cell(const hsn_cell_round& s, int64_t p) {
    if (!s.valid[p]) return -1;
    const int64_t c = s.cells[p];
    return c >= 0 && c < s.N ? static_cast<int>(c) : -1;
}
__device__ __forceinline__ int unit_of(const hsn_cell_round& s, int64_t p) {
    const int64_t j = s.units[p];
    return static_cast<int>(j < 0 ? 0 : (j >= s.M ? s.M - 1 : j));
}

__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// One 16 x 16 tile of A (16 rows in LDS, this lane's row at `a`) times B (kdim x 16; b(k) is
// this lane's column at reduction index k), kdim = 4 quarter. Lane l supplies A[l % 16][k] and
// B[k][l % 16] for one k of each 4-step (v_mfma_f32_16x16x4_f32's layout): here lane group
// g = l / 16 walks the quarter [g quarter, (g + 1) quarter) in order, which sums the same terms
// with A's row read contiguously. Returns D[4 g + r][l % 16] in element r. Every lane of the
// wavefront must call it (MFMA runs on the whole wavefront).
template <typename BLoad>
__device__ __forceinline__ v4f tile_product(const float* a, int quarter, int g, BLoad b) {
    const int k0 = g * quarter;
    const float* ag = a + k0;
    v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    int s = 0;
    for (; s + 8 <= quarter; s += 8) {
        float bv[8], av[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) bv[i] = b(k0 + s + i);
#pragma unroll
        for (int i = 0; i < 8; ++i) av[i] = ag[s + i];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[i], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i + 1], bv[i + 1], acc1, 0, 0, 0);
        }
    }
    for (; s < quarter; ++s)
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ag[s], b(k0 + s), acc0, 0, 0, 0);
    return acc0 + acc1;
}

// ---- front: messages, input, cell norm, gate ----------------------------------------------------
__global__ __launch_bounds__(kRoundThreads) void round_front(hsn_cell_round s) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int d = s.d, n = 4 * d, K = s.K, N = s.N, D = s.D;
    const int64_t P = int64_t(s.B) * K;
    const FrontLds L = front_lds(d);
    int* cell_of = reinterpret_cast<int*>(lds + L.cell);
    float* hbar = reinterpret_cast<float*>(lds + L.hbar);
    float* x = reinterpret_cast<float*>(lds + L.x);
    float* rms = reinterpret_cast<float*>(lds + L.rms);
    const int64_t p0 = int64_t(blockIdx.x) * kRows;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int lr = lane & 15, g = lane >> 4;
    const Work W = work_of(s.B, K, d, s.H);
    float* v_out = reinterpret_cast<float*>(static_cast<unsigned char*>(s.work) + W.v);
    float* gate_out = reinterpret_cast<float*>(static_cast<unsigned char*>(s.work) + W.gate);

    if (tid < kRows) cell_of[tid] = p0 + tid < P ? live_cell(s, p0 + tid) : -1;
    __syncthreads();

    // the input's state blocks and each slot's weighted source sum (edges in slot order)
    for (int e = tid; e < kRows * d; e += kRoundThreads) {
        const int pp = e / d, c = e % d;
        const int cell = cell_of[pp];
        float sum = 0.0f, uu = 0.0f, ee = 0.0f, hh = 0.0f;
        if (cell >= 0) {
            const int64_t r = (p0 + pp) / K;
            const float* hr = s.h + r * N * d;
            const int64_t* src = s.pad_src + int64_t(cell) * D;
            const float* w = s.edge_w + int64_t(cell) * D;
#pragma unroll 4
            for (int k = 0; k < D; ++k) {
                const int64_t j = src[k];
                const float hv = j >= 0 && j < N ? hr[j * d + c] : 0.0f;
                sum += w[k] * hv;
            }
            uu = s.u[r * d + c];
            ee = s.eps[r * d + c];
            hh = hr[int64_t(cell) * d + c];
        }
        hbar[pp * L.sh + c] = sum;
        x[pp * L.sx + c] = uu;
        x[pp * L.sx + d + c] = ee;
        x[pp * L.sx + 2 * d + c] = hh;
    }
    __syncthreads();

    // m = V hbar: B[k][col] = V[col][k]
    const int tiles_d = (d + 15) / 16;
    for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
        const int col = tile * 16 + lr;
        const bool ok = col < d;
        const float* vrow = s.V + int64_t(ok ? col : 0) * d;
        const v4f acc = tile_product(hbar + lr * L.sh, d / 4, g, [&](int k) {
            const float w = vrow[k];
            return ok ? w : 0.0f;
        });
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (ok) x[(4 * g + r) * L.sx + 3 * d + col] = acc[r];
    }
    __syncthreads();

    // the cell norm: 1 / sqrt(mean(x^2) + eps) a slot, a wavefront a slot
    for (int pp = wave; pp < kRows; pp += kRoundWaves) {
        float ss = 0.0f;
        for (int c = lane; c < n; c += kWave) {
            const float t = x[pp * L.sx + c];
            ss += t * t;
        }
        ss = group_sum<kWave>(ss);
        if (lane == 0) rms[pp] = rsqrtf(ss / static_cast<float>(n) + s.norm_eps);
    }
    __syncthreads();
    for (int e = tid; e < kRows * n; e += kRoundThreads) {
        const int pp = e / n, c = e % n;
        const float val = x[pp * L.sx + c] * rms[pp] * s.norm_w[c];
        x[pp * L.sx + c] = val;
        if (cell_of[pp] >= 0) v_out[(p0 + pp) * n + c] = val;
    }
    __syncthreads();

    // the gate: sigmoid(gate_w v + gate_b), B[k][col] = gate_w[col][k]
    for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
        const int col = tile * 16 + lr;
        const bool ok = col < d;
        const float* grow = s.gate_w + int64_t(ok ? col : 0) * n;
        const v4f acc = tile_product(x + lr * L.sx, d, g, [&](int k) {
            const float w = grow[k];
            return ok ? w : 0.0f;
        });
        const float bias = ok ? s.gate_b[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int pp = 4 * g + r;
            if (ok && cell_of[pp] >= 0) gate_out[(p0 + pp) * d + col] = act_sigmoid(acc[r] + bias);
        }
    }
}

// ---- units: the selected units' MLP, 64 hidden units a workgroup --------------------------------
__global__ __launch_bounds__(kRoundThreads) void round_units(hsn_cell_round s) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int d = s.d, n = 4 * d, M = s.M, H = s.H;
    const int P = s.B * s.K;
    const UnitsLds L = units_lds(P, d);
    uint8_t* ucache = lds + L.ucache;
    int* rows = reinterpret_cast<int*>(lds + L.rows);
    int* meta = reinterpret_cast<int*>(lds + L.meta);
    float* vs = reinterpret_cast<float*>(lds + L.v);
    float* act = reinterpret_cast<float*>(lds + L.act);
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const int lr = lane & 15, g = lane >> 4;
    const int chunk = blockIdx.y;
    const Work W = work_of(s.B, s.K, d, H);
    const float* v_in = reinterpret_cast<const float*>(static_cast<unsigned char*>(s.work) + W.v);
    float* part = reinterpret_cast<float*>(static_cast<unsigned char*>(s.work) + W.part);

    for (int q = tid; q < P; q += kRoundThreads)
        ucache[q] = live_cell(s, q) >= 0 ? static_cast<uint8_t>(unit_of(s, q)) : uint8_t(0xff);
    __syncthreads();
    // which unit's which row tile: units in order, each with ceil(count / 16) tiles
    if (wave == 0) {
        int before = 0, unit = -1, tile = 0;
        for (int j = 0; j < M && unit < 0; ++j) {
            int cnt = 0;
            for (int q0 = 0; q0 < P; q0 += kWave)
                cnt += __popcll(ballot(q0 + lane < P && ucache[q0 + lane] == j));
            const int tiles = (cnt + kRows - 1) / kRows;
            if (static_cast<int>(blockIdx.x) < before + tiles) {
                unit = j;
                tile = blockIdx.x - before;
            }
            before += tiles;
        }
        if (lane < kRows) rows[lane] = -1;
        if (unit >= 0) {
            const int first = tile * kRows;
            int base = 0;
            for (int q0 = 0; q0 < P && base < first + kRows; q0 += kWave) {
                const int q = q0 + lane;
                const bool mine = q < P && ucache[q] == unit;
                const uint64_t m = ballot(mine);
                const int rank = base + lanes_below(m);
                if (mine && rank >= first && rank < first + kRows) rows[rank - first] = q;
                base += __popcll(m);
            }
        }
        if (lane == 0) meta[0] = unit;
    }
    __syncthreads();
    const int j = meta[0];
    if (j < 0) return;  // past the last row tile (uniform)

    for (int e = tid; e < kRows * n; e += kRoundThreads) {
        const int pp = e / n, c = e % n;
        const int q = rows[pp];
        vs[pp * L.sv + c] = q >= 0 ? v_in[int64_t(q) * n + c] : 0.0f;
    }
    __syncthreads();

    // hidden = v W1_j + b1_j on this chunk's 64 columns, a 16-column tile a wavefront
    {
        const int hc = wave * 16 + lr;
        const int col = chunk * kChunk + hc;
        const bool ok = col < H;
        const float* w1 = s.W1 + int64_t(j) * n * H + (ok ? col : 0);
        const v4f acc = tile_product(vs + lr * L.sv, d, g, [&](int k) {
            const float w = w1[int64_t(k) * H];
            return ok ? w : 0.0f;
        });
        const float bias = ok ? s.b1[int64_t(j) * H + col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) act[(4 * g + r) * L.sa + hc] = ok ? gelu_erf(acc[r] + bias) : 0.0f;
    }
    __syncthreads();

    // this chunk's share of F = act W2_j: B[k][col] = W2[j][chunk 64 + k][col]
    const int tiles_d = (d + 15) / 16;
    const int h0 = chunk * kChunk;
    for (int tile = wave; tile < tiles_d; tile += kRoundWaves) {
        const int col = tile * 16 + lr;
        const bool ok = col < d;
        const float* w2 = s.W2 + (int64_t(j) * H + h0) * d + (ok ? col : 0);
        const v4f acc = tile_product(act + lr * L.sa, kChunk / 4, g, [&](int k) {
            const int kk = h0 + k < H ? k : H - 1 - h0;  // rows past H read a valid row, unused
            const float w = w2[int64_t(kk) * d];
            return ok && h0 + k < H ? w : 0.0f;
        });
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = rows[4 * g + r];
            if (ok && q >= 0) part[(int64_t(chunk) * P + q) * d + col] = acc[r];
        }
    }
}

// ---- back: W_out, candidate, update, q, h_sel; the other cells' copy and the tick --------------
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
    }
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
    const Work W = work_of(s.B, K, d, s.H);
    const float* gate = reinterpret_cast<const float*>(static_cast<unsigned char*>(s.work) + W.gate);
    const float* part = reinterpret_cast<const float*>(static_cast<unsigned char*>(s.work) + W.part);
    const int chunks = chunks_of(s.H);

    // F = the chunks' shares in chunk order + b2_j; alpha before W_out without the candidate norm
    for (int e = tid; e < L.k16 * d; e += kRoundThreads) {
        const int k = e / d, xc = e % d;
        float val = 0.0f;
        if (kcell[k] >= 0) {
            const int64_t p = r * K + k;
            float f = 0.0f;
            for (int c = 0; c < chunks; ++c) f += part[(int64_t(c) * P + p) * d + xc];
            f += s.b2[int64_t(kunit[k]) * d + xc];
            val = s.cand_norm ? f : s.alpha[p] * f;
        }
        o[k * L.so + xc] = val;
    }
    __syncthreads();

    // pre = W_out o: B[k][col] = W_out[col][k], tiles over (slot tile, column tile)
    const int tiles_d = (d + 15) / 16;
    const int lr = lane & 15, g = lane >> 4;
    for (int tile = wave; tile < (L.k16 / 16) * tiles_d; tile += kRoundWaves) {
        const int rt = tile / tiles_d, ct = tile % tiles_d;
        const int col = ct * 16 + lr;
        const bool ok = col < d;
        const float* wrow = s.W_out + int64_t(ok ? col : 0) * d;
        const v4f acc = tile_product(o + (rt * 16 + lr) * L.so, d / 4, g, [&](int k) {
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
            const int64_t p = r * K + k;
            const float y = pre[k * L.so + xc];
            const float value = s.cand_norm ? s.alpha[p] * (y * scale[k] * s.cand_w[xc]) : y;
            const float c = tanhf(value);
            const float old = h[int64_t(cell) * d + xc];
            const float b = gate[p * d + xc];
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
        s.q_new[r * d + xc] = s.q[r * d + xc] + sum / static_cast<float>(N);
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
                "cell round: more than 16384 slots (B K) a position");
    HSN_REQUIRE(front_lds(s->d).bytes <= kMaxLds && units_lds(s->B * s->K, s->d).bytes <= kMaxLds,
                HSN_ERR_INVALID_ARGUMENT, "cell round: 16 slots' inputs exceed 160 KiB of LDS");
    HSN_REQUIRE(back_lds(s->K, s->d).bytes <= kMaxLds, HSN_ERR_INVALID_ARGUMENT,
                "cell round: a row's slots (8 K d bytes) exceed 160 KiB of LDS");
    const int64_t P = int64_t(s->B) * s->K;
    HSN_REQUIRE(check_elems({int64_t(s->B) * s->N * s->d, P * 4 * s->d,
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
    HSN_REQUIRE(reinterpret_cast<uintptr_t>(s->work) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(s->h) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(s->h_new) % 16 == 0,
                HSN_ERR_INVALID_ARGUMENT, "cell round: work, h and h_new must be 16-byte aligned");
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
    launch(round_front, dim3(tiles), front_lds(s.d).bytes, st, s);
    launch(round_units, dim3(tiles + static_cast<unsigned>(s.M), chunks_of(s.H)),
           units_lds(P, s.d).bytes, st, s);
    launch(round_back, dim3(s.B, 1 + (s.N + kCopyCells - 1) / kCopyCells),
           back_lds(s.K, s.d).bytes, st, s);
    HSN_ABI_END
}
