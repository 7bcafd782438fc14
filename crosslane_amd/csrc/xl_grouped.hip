// CDNA4 (gfx950) grouped routed-expert path: T tokens, each with its own k
// picks, reading every touched expert's weights once per 16 of its (token,
// pick) pairs. The result is that of T independent layer calls
// (WarmRedirect::warm_compute_many per token, engine/strata/warm/runtime.hpp:13,
// then the fixed-order join of runtime.cpp:183-188): per (row, pair) the same
// exact integer block partials and the same fp16(d) * d_x fma over blocks in
// block order as the row kernels.
//
//   bucket_kernel    one workgroup: pairs bucketed by expert id into tasks of
//                    at most 16 pairs of one expert
//   q8k_rows_kernel  Q8_K (q8k_core.hpp:30-38) of token rows (x) and pair rows
//                    (h), written in the operand order of the MFMA kernels
//   gu_kernel        gate/up + SwiGLU of every task (IQ2_XXS)
//   dn_kernel        down of every task (IQ2_XS)
//   gcombine_kernel  fixed-order combine per token, + shared
//
// MFMA: v_mfma_i32_16x16x32_i8 with M = pairs, N = weight rows, K = the 32
// weights of one sub-block. Lane l supplies A[l % 16][8 (l / 16) .. + 7] (8
// quants of pair l % 16), B[8 (l / 16) .. + 7][l % 16] (grid entry l / 16 of
// row l % 16: 8 weights) and receives D[4 (l / 16) + r][l % 16], r = 0..3. The
// lane that decodes a row's entry therefore also holds that row's outputs and
// applies the row's sub-block scale (2s + 1) to them as integers: the block
// partials are exact. Any K order works as long as A and B agree, which the
// chunk-major activation layouts below guarantee.
//
// Weights stream from HBM through registers: each wave loads its 16 rows' next
// block while it computes the current one, and touches the line four blocks
// ahead with one dword per row so that it is in L2 when the real loads come.
// The texture data path costs one cycle per cache access, and a quad of lanes
// makes one access only when it reads 64 contiguous bytes: so each lane loads
// just the 16 B of its row's block that it decodes (the entries then move
// between lane groups by permlane swaps), activations are laid out so that a
// quad's four slots are adjacent, and the small per-block scales are staged in
// LDS once per work item instead of being loaded by every wave.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "xl_dev.hpp"
#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace xl::dev {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;   // pairs per task (the MFMA M dimension)
// Expanded codebook tables (layer_tables() in xl_api.cpp): 128 sign entries of
// 16 B (byte mask, then the mask's low bits), the IQ2_XXS grid (256 x 8 B), the
// IQ2_XS grid (512 x 8 B).
constexpr int kTabSgn = 0, kTabXXS = 2048, kTabXS = 4096;

// LDS of the MFMA kernels: grid entries as 16 B (g, -g) in C copies per entry
// (lane copy = lane % C, so the 16 lanes of one ds_read_b128 pass never share
// a bank), sign masks as 8 B in 32 copies (the 32 lanes of one ds_read_b64 pass
// never share a bank) indexed by a whole byte whose top bit is not a sign bit.
constexpr int kL_GRID = 0, kL_SGN = 65536, kL_TAB = 131072;
// Per work item, staged once by the workgroup (each wave would otherwise issue
// these small loads every block): the 16 pairs' activation block scales
// [block][pair] (f32), then the item's rows' fp16 block scales [row][block]
// for each matrix (NW x 16 rows), then (down) the rows' IQ2_XS scale bytes
// [row][block][8].
// Blocks per row these regions hold: gate/up rows of dim <= kMaxRowK, down
// rows of ff <= 4096.
constexpr int kGuNb = kMaxRowK / 256, kDnNb = 16;
constexpr int kL_PD = kL_TAB;
constexpr int kL_RDG = kL_PD + 16 * kGuNb * 4;     // gate/up: 2 planes of `rows` rows x kGuNb fp16 scales
constexpr int gu_lds_bytes(int rows) { return kL_RDG + 2 * rows * kGuNb * 2; }
constexpr int kL_RDD = kL_PD + 16 * kDnNb * 4;     // down: `rows` rows x kDnNb fp16 scales, then scale bytes
constexpr int dn_rs(int rows) { return kL_RDD + rows * kDnNb * 2; }
constexpr int dn_lds_bytes(int rows) { return dn_rs(rows) + rows * kDnNb * 8; }
static_assert(gu_lds_bytes(12 * 16) <= 160 * 1024 && dn_lds_bytes(12 * 16) <= 160 * 1024, "LDS budget");
constexpr int kCopiesXXS = 16;   // 256 entries x 256 B: the entry byte lands in address byte 1
constexpr int kCopiesXS = 8;     // 512 entries x 128 B: the 9-bit entry lands at address bit 7

// Values every lane of the wave holds alike, moved to scalar registers (buffer
// descriptors built from them stay scalar: no waterfall loops).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const uint8_t* uni(const uint8_t* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<const uint8_t*>((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ int4 task_at(const int4* tasks, int i) {
    const int4 t = tasks[i];
    return make_int4(uni(t.x), uni(t.y), uni(t.z), 0);
}
__device__ __forceinline__ MatRef mat_at(const ExpertDesc* d, int e, int role) {
    const MatRef m = d[e].m[role];
    MatRef u;
    u.base = uni(m.base);
    u.off1 = (uint64_t(uint32_t(uni(int(m.off1 >> 32)))) << 32) | uint32_t(uni(int(uint32_t(m.off1))));
    u.off2 = (uint64_t(uint32_t(uni(int(m.off2 >> 32)))) << 32) | uint32_t(uni(int(uint32_t(m.off2))));
    u.type = uni(m.type);
    u.nb = uni(m.nb);
    return u;
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t x, uint32_t y) { return (m & x) | (~m & y); }
__device__ __forceinline__ long pack64(uint32_t lo, uint32_t hi) {
    return static_cast<long>((uint64_t(hi) << 32) | lo);
}
__device__ __forceinline__ v4i mfma(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int mad24(int a, int b, int c) {   // v_mad_i32_i24
    // the opaque result keeps the add from merging into a v_add3 (mul + add3 per
    // pair of terms instead of one mad each)
    int r = __mul24(a, b) + c;
    asm volatile("" : "+v"(r));
    return r;
}
// Bytewise negation of grid bytes (all in 1..127, so no byte borrows).
__device__ __forceinline__ uint64_t neg_grid(uint64_t g) { return ~g + 0x0101010101010101ull; }

// Sign tables: 256 rows (row r = sign entry r & 127) x 32 copies x 8 B.
__device__ __forceinline__ void fill_signs(uint8_t* lds, const uint64_t* tab, int t, int nt) {
    for (int i = t; i < 256 * 32; i += nt)
        *reinterpret_cast<uint64_t*>(lds + kL_SGN + 8 * i) = tab[kTabSgn / 8 + 2 * ((i >> 5) & 127)];
}
// Grid tables: E entries x C copies x 16 B (g, -g).
template <int E, int C>
__device__ __forceinline__ void fill_grid(uint8_t* lds, const uint64_t* grid, int t, int nt) {
    for (int i = t; i < E * C; i += nt) {
        const uint64_t g = grid[i / C], n = neg_grid(g);
        *reinterpret_cast<uint4*>(lds + kL_GRID + 16 * i) =
            make_uint4(uint32_t(g), uint32_t(g >> 32), uint32_t(n), uint32_t(n >> 32));
    }
}

// ---------------------------------------------------------------------------
// Buckets: counts per expert in LDS, one scan of pairs and tasks, then each
// valid pair takes a slot of its expert's tasks (task i: slots 16 i .. + 15).
// The slot order inside an expert varies run to run; no result depends on it
// (every output of a pair is computed from that pair's operands only, in a
// fixed order).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void bucket_kernel(GroupArgs a) {
    __shared__ int cnt[kGroupMaxExperts];
    __shared__ int cur[kGroupMaxExperts];
    __shared__ int part[2 * 1024];
    const int t = threadIdx.x, P = a.T * a.k, E = a.n_experts;
    for (int e = t; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = a.ids[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        else atomicOr(a.err, kDevErrExpertId);
    }
    __syncthreads();
    const int per = (E + 1023) / 1024, e0 = min(E, t * per), e1 = min(E, e0 + per);
    int st = 0;
    for (int e = e0; e < e1; ++e) st += (cnt[e] + kTile - 1) / kTile;
    part[t] = st;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {   // inclusive scan of tasks
        const int v = t >= off ? part[t - off] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    int bt = part[t] - st;
    for (int e = e0; e < e1; ++e) {
        const int c = cnt[e];
        for (int i = 0; i * kTile < c; ++i)
            a.tasks[bt + i] = make_int4(e, kTile * (bt + i), min(kTile, c - kTile * i), 0);
        cur[e] = kTile * bt;   // the expert's first slot; its pairs fill its tasks' slots in turn
        bt += (c + kTile - 1) / kTile;
    }
    if (t == 1023) *a.n_tasks = part[1023];
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = a.ids[p];
        int slot = -1;
        if (e >= 0 && e < E) {
            slot = atomicAdd(&cur[e], 1);   // consecutive per expert: its tasks' slots have no gaps before the last
            a.order[slot] = p;
        }
        a.pos[p] = slot;
    }
}

// ---------------------------------------------------------------------------
// Q8_K of 256-value blocks of rows, one wave per block, written to the slots of
// the row's pairs (ROWS_X: a token row goes to its k pairs' slots; ROWS_H: a
// pair row to its slot; bad ids have none) in the operand order of the MFMA
// kernels. Task i's slots form one region of nb * 4 KiB; in it, per block b,
// the 16-B piece i of chunk e (the 8 quants of entry e of sub-blocks 2i and
// 2i + 1) of slot s sits at ((4 b + i) * 4 + e) * 256 + 16 s, so that four lanes
// of consecutive slots read 64 contiguous bytes.
// ---------------------------------------------------------------------------
// The j-th pair of a task (slot 16 i + j) sits at tile position 4 (j % 4) + j / 4
// (M index of the MFMAs; the map is its own inverse): the lane holding M rows
// 4 e + r, r = 0..3, gets pairs 4 r + e, so a task of n pairs has results only
// in the lanes' first ceil(n / 4) output registers.
__device__ __forceinline__ int tile_pos(int j) { return ((j & 3) << 2) | (j >> 2); }
__device__ __forceinline__ size_t slot_off(int slot, int nb, int blk, int piece, int chunk) {
    return size_t(slot >> 4) * size_t(nb) * 4096 +
           size_t(((4 * blk + piece) * 4 + chunk) * 256 + 16 * tile_pos(slot & 15));
}
enum { ROWS_X = 0, ROWS_H = 1 };
// trace (null outside the parity trace): the row's blocks also as 292-byte Q8_K
// blocks, row-major (a token's for ROWS_X, a pair's for ROWS_H).
template <int MODE, bool TR>
__global__ __launch_bounds__(256) void q8k_rows_kernel(const float* __restrict__ src, int rows, int nb,
                                                       int8_t* __restrict__ q, float* __restrict__ d,
                                                       const int32_t* __restrict__ pos, int k,
                                                       int* __restrict__ err, uint8_t* __restrict__ trace) {
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= rows * nb) return;   // wave-uniform
    const int row = b / nb, blk = b - row * nb;
    if (MODE == ROWS_H && pos[row] < 0) return;
    const int lane = threadIdx.x & 63;
    const float4 v4 = reinterpret_cast<const float4*>(src + size_t(b) * 256)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    const Q8Lane r = q8k_lane(v, lane);
    if (!r.finite && lane == 0) atomicOr(err, kDevErrNonFinite);
    const int c = lane >> 3, e = (lane >> 1) & 3, j = 8 * (c & 1) + 4 * (lane & 1);   // values 4 lane .. + 3
    const int np = MODE == ROWS_X ? k : 1;
    for (int i = 0; i < np; ++i) {
        const int slot = pos[MODE == ROWS_X ? row * k + i : row];
        if (slot >= 0) *reinterpret_cast<uint32_t*>(q + slot_off(slot, nb, blk, c >> 1, e) + j) = r.packed;
    }
    if (lane == 0) d[b] = r.d;
    if constexpr (TR) {
        if (trace) trace_q8_block(trace + size_t(b) * 292, r.d, r.packed, lane);
    }
}

// Keeps a value alive without storing it (the L2 line touches).
__device__ __forceinline__ void sink(uint32_t& acc, uint32_t v) { acc ^= v; }

// Buffer loads: the base in a scalar descriptor, the per-lane byte offset in
// voffset, a uniform plane offset in soffset.
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t so = 0) {
    const v4u32 q = __builtin_amdgcn_raw_buffer_load_b128(r, v, so, 0);
    return make_uint4(q.x, q.y, q.z, q.w);
}
__device__ __forceinline__ uint2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t so = 0) {
    const v2u32 q = __builtin_amdgcn_raw_buffer_load_b64(r, v, so, 0);
    return make_uint2(q.x, q.y);
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t so = 0) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, v, so, 0);
}
__device__ __forceinline__ uint16_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t v, uint32_t so = 0) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, v, so, 0);
}

// One block's operands for one wave.
struct GuOps {
    uint4 g, u, a[4];   // 16-B part e4 of the row's gate / up block, the lane's activation chunk
};

// Exchanges across the four 16-lane groups (e4 = lane / 16) of a wave.
__device__ __forceinline__ void swap32(uint32_t& x, uint32_t& y) {   // lanes 32.. of x <-> lanes ..31 of y
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    x = r[0];
    y = r[1];
}
__device__ __forceinline__ void swap16(uint32_t& x, uint32_t& y) {   // odd groups of x <-> even groups of y
    const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    x = r[0];
    y = r[1];
}
// v[j] of group g -> v[g] of group j, lane by lane within the groups.
__device__ __forceinline__ void xpose4(uint32_t (&v)[4]) {
    swap32(v[0], v[2]);
    swap32(v[1], v[3]);
    swap16(v[0], v[1]);
    swap16(v[2], v[3]);
}
// Every group's byte x (placed at byte e4 by the caller) in every group.
__device__ __forceinline__ uint32_t gather4(uint32_t x) {
    uint32_t y = x;
    swap32(x, y);
    x |= y;
    y = x;
    swap16(x, y);
    return x | y;
}

// IQ2_XXS block of the MFMA lane (col, e4) from 16-B parts: lane (col, g) loaded
// bytes 16 g .. + 15 of row col's block (sub-blocks 2g and 2g + 1: grid bytes,
// then aux bytes = 7 sign bits | scale bit k in byte k). Afterwards u[j] holds
// {grid, aux} bytes of entry e4 of sub-blocks 2j (bytes 0, 1) and 2j + 1 (bytes
// 2, 3), and byte j of ls[c & 1] holds sub-block c = 2j + (c & 1)'s factor
// 2 s + 1 (s its 4-bit scale).
struct XxsLane {
    uint32_t u[4], ls[2];
};
__device__ __forceinline__ XxsLane xxs_lane(const uint4& w, int e4) {
    const uint32_t p01 = perm(w.y, w.x, 0x05010400u), p01b = perm(w.y, w.x, 0x07030602u);
    const uint32_t p23 = perm(w.w, w.z, 0x05010400u), p23b = perm(w.w, w.z, 0x07030602u);
    XxsLane r;
    r.u[0] = perm(p23, p01, 0x05040100u);    // entry 0 of both sub-blocks
    r.u[1] = perm(p23, p01, 0x07060302u);
    r.u[2] = perm(p23b, p01b, 0x05040100u);
    r.u[3] = perm(p23b, p01b, 0x07060302u);
    xpose4(r.u);
    const uint32_t sa = __builtin_amdgcn_udot4((w.y >> 7) & 0x01010101u, 0x08040201u, 0u, false);
    const uint32_t sb = __builtin_amdgcn_udot4((w.w >> 7) & 0x01010101u, 0x08040201u, 0u, false);
    const uint32_t s = gather4((sa | (sb << 4)) << (8 * e4));   // sub-block c's scale at bits 4c .. 4c + 3
    r.ls[0] = ((s << 1) & 0x1E1E1E1Eu) | 0x01010101u;
    r.ls[1] = ((s >> 3) & 0x1E1E1E1Eu) | 0x01010101u;
    return r;
}
struct DnOps {
    uint4 q, a[4];      // 16-B part e4 of the row's down block, the lane's activation chunk
};

// Stages one item's pair scales (scl: one f32 per (pair row, block), pairs of
// the task's order slots) and `mats` planes of fp16 row scales (rows rows from
// row0, nb per row, contiguous in each plane) into LDS, after a barrier.
// The planes go to LDS at rd, `mstride` bytes apart.
template <int NT>
__device__ __forceinline__ void stage_item(uint8_t* lds, const GroupArgs& a, const int4& tk, const float* scl, int per_pair,
                                           int nb, const uint8_t* const* planes, int mats, int row0, int rows, int t,
                                           int rd, int mstride) {
    __syncthreads();   // every wave is done with the previous item's staging
    for (int i = t; i < 16 * nb; i += NT) {
        const int pos = i & 15, blk = i >> 4;   // tile position pos holds the task's pair tile_pos(pos)
        const int p = a.order[tk.y + min(tile_pos(pos), tk.z - 1)];
        reinterpret_cast<float*>(lds + kL_PD)[i] = scl[size_t(per_pair ? p : p / a.k) * nb + blk];
    }
    const int chunks = rows * nb * 2 / 16;   // 16-byte pieces of one plane's rows
    for (int i = t; i < mats * chunks; i += NT) {
        const int m = i / chunks, c = i - m * chunks;
        const uint4 v = reinterpret_cast<const uint4*>(planes[m] + size_t(row0) * nb * 2)[c];
        *reinterpret_cast<uint4*>(lds + rd + m * mstride + 16 * c) = v;
    }
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU. Work item = (task, group of NW * 16 rows); wave wv owns
// rows 16 wv .. + 15 of the group in gate and up.
// ---------------------------------------------------------------------------
// TR: also write each pair's block integers (GroupArgs::tint).
template <int NW, bool TR>
__global__ __launch_bounds__(NW * 64, 1) void gu_kernel(GroupArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[gu_lds_bytes(NW * 16)];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    fill_grid<256, kCopiesXXS>(lds, a.tables + kTabXXS / 8, t, NW * 64);
    fill_signs(lds, a.tables, t, NW * 64);
    __syncthreads();

    const int col = lane & 15, e4 = lane >> 4;
    const int nb = a.dim / 256, groups = a.ff / (NW * 16);
    const int items = uni(*a.n_tasks) * groups;
    const uint32_t lo_g = uint32_t(lane & (kCopiesXXS - 1)) << 4;        // kL_GRID = 0
    const uint32_t lo_s = (uint32_t(lane & 31) << 3) | (1u << 16);       // kL_SGN = 1 << 16
    uint32_t sunk = 0;
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int task = item / groups, grp = item - task * groups;
        const int4 tk = task_at(a.tasks, task);
        const int row = grp * NW * 16 + wv * 16 + col;
        // A operand: slot col of the task (past its pairs: unused slot memory, whose
        // outputs are discarded), the lane's chunk e4, block 0
        const uint32_t va = uint32_t(slot_off(tk.y, nb, 0, 0, e4) + 16 * col);
        int po[4];   // the pairs of the lane's four outputs (tile positions 4 e4 + r)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = 4 * r + e4;
            po[r] = j < tk.z ? a.order[tk.y + j] : -1;
        }
        const MatRef G = mat_at(a.descs, tk.x, 0), U = mat_at(a.descs, tk.x, 1);
        {
            const uint8_t* planes[2] = {G.base + G.off1, U.base + U.off1};
            stage_item<NW * 64>(lds, a, tk, a.xd, 0, nb, planes, 2, grp * NW * 16, NW * 16, t, kL_RDG,
                                NW * 16 * kGuNb * 2);
        }
        const __amdgpu_buffer_rsrc_t rg = rsrc(G.base), ru = rsrc(U.base), rx = rsrc(a.xq);
        const uint32_t vq = uint32_t(row * nb) * 64u;
        auto load = [&](GuOps& o, int blk) {
            o.g = ld128(rg, vq + 64u * blk + 16u * e4);
            o.u = ld128(ru, vq + 64u * blk + 16u * e4);
#pragma unroll
            for (int i = 0; i < 4; ++i) o.a[i] = ld128(rx, va + 4096u * blk + 1024u * i);
        };
        auto touch = [&](int blk) { return ld32(rg, vq + 64u * blk) ^ ld32(ru, vq + 64u * blk); };
        // RR: output registers that can hold a pair (2 for tasks of at most 8 pairs, else 4)
        auto run = [&]<int RR>() {
            float accg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            // Sub-block c of a matrix: its grid entry (g, -g) and sign mask from LDS,
            // then B = signed entry, one MFMA, the row's (2s + 1) on the RR outputs.
            // All eight gate lookups are issued first; each up lookup is issued as a
            // gate one is consumed, so about seven are in flight throughout.
            struct Look { uint4 g; uint2 m; };
            auto look = [&](const XxsLane& X, int c) {   // grid byte -> address byte 1, then the aux byte
                const uint32_t w = X.u[c >> 1], h = uint32_t(c & 1) * 2u;
                Look L;
                L.g = *reinterpret_cast<const uint4*>(lds + perm(w, lo_g, 0x0C020000u | ((4u + h) << 8)));
                L.m = *reinterpret_cast<const uint2*>(lds + perm(w, lo_s, 0x0C020000u | ((5u + h) << 8)));
                return L;
            };
            auto prod = [&](const Look& L, long A) {
                return mfma(A, pack64(bfi(L.m.x, L.g.z, L.g.x), bfi(L.m.y, L.g.w, L.g.y)), v4i{0, 0, 0, 0});
            };
            auto scale = [&](const v4i& C, const XxsLane& X, int c, int (&bi)[4]) {
                const int ls = int(__builtin_amdgcn_ubfe(X.ls[c & 1], 8 * (c >> 1), 8));
#pragma unroll
                for (int r = 0; r < RR; ++r) bi[r] = mad24(ls, C[r], bi[r]);
            };
            const uint16_t* sdg = reinterpret_cast<const uint16_t*>(lds + kL_RDG) + (wv * 16 + col) * nb;
            const uint16_t* sdu = sdg + NW * 16 * kGuNb;
            int blk_c = 0;   // block the next compute() handles
            auto compute = [&](const GuOps& o) {
                const int b = blk_c++;
                int big[4] = {0, 0, 0, 0}, biu[4] = {0, 0, 0, 0};
                long A[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const uint32_t* av = reinterpret_cast<const uint32_t*>(o.a) + 2 * c;
                    A[c] = pack64(av[0], av[1]);
                }
                const XxsLane XG = xxs_lane(o.g, e4), XU = xxs_lane(o.u, e4);
                Look L[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) L[c] = look(XG, c);
                // step i < 8: gate sub-block i, else up sub-block i - 8; each step's
                // MFMA is issued before the previous step's multiply-adds read theirs
                v4i C[16];
#pragma unroll
                for (int i = 0; i <= 16; ++i) {
                    if (i < 8) {
                        C[i] = prod(L[i], A[i]);
                        L[i] = look(XU, i);
                    } else if (i < 16) {
                        C[i] = prod(L[i - 8], A[i - 8]);
                    }
                    if (i > 8) scale(C[i - 1], XU, i - 9, biu);
                    else if (i > 0) scale(C[i - 1], XG, i - 1, big);
                }
                if constexpr (TR) {   // pair po[r]'s block integers of this lane's row
                    const size_t rec = 2 * size_t(a.ff) * nb + size_t(a.dim) * (a.ff / 256);
#pragma unroll
                    for (int r = 0; r < RR; ++r)
                        if (a.tint && po[r] >= 0) {
                            const size_t o = size_t(po[r]) * rec + size_t(row) * nb + size_t(b);
                            a.tint[o] = big[r];
                            a.tint[o + size_t(a.ff) * nb] = biu[r];
                        }
                }
                const float dgf = h2f(sdg[b]), duf = h2f(sdu[b]);
                const float4 xd4 = *reinterpret_cast<const float4*>(lds + kL_PD + 64 * b + 16 * e4);
                const float xd[4] = {xd4.x, xd4.y, xd4.z, xd4.w};
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    accg[r] = fmaf(__fmul_rn(dgf, xd[r]), float(big[r]), accg[r]);
                    accu[r] = fmaf(__fmul_rn(duf, xd[r]), float(biu[r]), accu[r]);
                }
            };
            // Two operand sets alternate over a 4-step unrolled loop (no register
            // copies, so no wait ever covers a load issued in the same step); line
            // touches four blocks ahead in four fixed registers.
            // A row's blocks 2j and 2j + 1 share a 128-byte line: one touch per line.
            GuOps s0, s1;
            load(s0, 0);
            uint32_t t0 = touch(min(1, nb - 1)), t2 = touch(min(3, nb - 1));
            for (int b = 0; b < nb; b += 4) {
                load(s1, min(b + 1, nb - 1));
                sink(sunk, t0);
                t0 = touch(min(b + 5, nb - 1));
                __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the compute
                compute(s0);
                load(s0, min(b + 2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 1 < nb) compute(s1);
                load(s1, min(b + 3, nb - 1));
                sink(sunk, t2);
                t2 = touch(min(b + 7, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 2 < nb) compute(s0);
                load(s0, min(b + 4, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 3 < nb) compute(s1);
            }
            sink(sunk, t0 ^ t2);
#pragma unroll
            for (int r = 0; r < RR; ++r)
                if (po[r] >= 0)
                    a.h[size_t(po[r]) * a.ff + row] =
                        silu_mul3(__fmul_rn(0.125f, accg[r]), __fmul_rn(0.125f, accu[r]), a.lim);
        };
        __syncthreads();   // the item's scales are staged
        if (tk.z <= 8) run.template operator()<2>();
        else run.template operator()<4>();
    }
    if (sunk == 0x9e3779b9u && lane == 64) a.h[0] = 0.0f;   // never true (lane < 64): keeps the touches
}

// IQ2_XS block of the MFMA lane (col, e4) from 16-B parts, as xxs_lane: u[j]
// holds the 16-bit code (9-bit grid index at bits 7..15, sign bits 0..6) of
// entry e4 of sub-block 2j (low half) and 2j + 1 (high half).
__device__ __forceinline__ void xs_lane(const uint4& w, uint32_t (&u)[4]) {
    u[0] = perm(w.z, w.x, 0x05040100u);
    u[1] = perm(w.z, w.x, 0x07060302u);
    u[2] = perm(w.w, w.y, 0x05040100u);
    u[3] = perm(w.w, w.y, 0x07060302u);
    xpose4(u);
}

// ---------------------------------------------------------------------------
// down. Work item = (task, group of NW * 16 output rows; the last group of a
// task holds what is left of dim, whole waves of 16 rows, and the waves past
// it only join the item's barriers). IQ2_XS keeps a scale
// nibble per 16 weights (entries 0, 1 of a sub-block: ls1; entries 2, 3: ls2):
// per sub-block one MFMA over all 32 weights (C) and one with entries 2, 3 of B
// zeroed (C1), then ls1 C1 + ls2 (C - C1) as ls2 C + (ls1 - ls2) C1, exactly.
// ---------------------------------------------------------------------------
template <int NW, bool TR>
__global__ __launch_bounds__(NW * 64, 1) void dn_kernel(GroupArgs a) {
    constexpr int R = NW * 16;   // rows per item
    constexpr int kL_RS = dn_rs(R);
    static_assert(dn_lds_bytes(R) <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(16))) uint8_t lds[dn_lds_bytes(R)];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    fill_grid<512, kCopiesXS>(lds, a.tables + kTabXS / 8, t, NW * 64);
    fill_signs(lds, a.tables, t, NW * 64);
    __syncthreads();

    const int col = lane & 15, e4 = lane >> 4;
    const int nb = a.ff / 256, groups = (a.dim + R - 1) / R;
    const int items = uni(*a.n_tasks) * groups;
    const uint32_t lo_x = uint32_t(lane & (kCopiesXS - 1)) << 4;        // kL_GRID = 0
    const uint32_t lo_s = (uint32_t(lane & 31) << 3) | (1u << 16);      // kL_SGN = 1 << 16
    const uint32_t mk = e4 < 2 ? ~0u : 0u;                               // lanes of entries 0, 1
    uint32_t sunk = 0;
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int task = item / groups, grp = item - task * groups;
        const int4 tk = task_at(a.tasks, task);
        const int row0 = grp * R, rows = min(R, a.dim - row0);   // rows: a multiple of 16
        const int row = row0 + wv * 16 + col;
        const uint32_t va = uint32_t(slot_off(tk.y, nb, 0, 0, e4) + 16 * col);   // as in gu_kernel
        int po[4];   // the pairs of the lane's four outputs (tile positions 4 e4 + r)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = 4 * r + e4;
            po[r] = j < tk.z ? a.order[tk.y + j] : -1;
        }
        const MatRef D = mat_at(a.descs, tk.x, 2);
        {
            const uint8_t* planes[1] = {D.base + D.off2};
            stage_item<NW * 64>(lds, a, tk, a.hd, 1, nb, planes, 1, row0, rows, t, kL_RDD, 0);
            const int chunks = rows * nb * 8 / 16;   // the rows' IQ2_XS scale bytes
            for (int i = t; i < chunks; i += NW * 64)
                *reinterpret_cast<uint4*>(lds + kL_RS + 16 * i) =
                    reinterpret_cast<const uint4*>(D.base + D.off1 + size_t(row0) * nb * 8)[i];
        }
        const __amdgpu_buffer_rsrc_t rd = rsrc(D.base), rh = rsrc(a.hq);
        const uint32_t vq = uint32_t(row * nb) * 64u;
        auto load = [&](DnOps& o, int blk) {
            o.q = ld128(rd, vq + 64u * blk + 16u * e4);
#pragma unroll
            for (int i = 0; i < 4; ++i) o.a[i] = ld128(rh, va + 4096u * blk + 1024u * i);
        };
        auto touch = [&](int blk) { return ld32(rd, vq + 64u * blk); };
        // RR: output registers that can hold a pair (ceil(pairs / 4), rounded up to 2, 3 or 4)
        auto run = [&]<int RR>() {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            const int rl = wv * 16 + col;   // the lane's row within the item
            int blk_c = 0;                   // block the next compute() handles
            auto compute = [&](const DnOps& o) {
                const int b = blk_c++;
                const uint2 sc = *reinterpret_cast<const uint2*>(lds + kL_RS + 8 * (rl * nb + b));
                // Scale byte c holds nibbles lo (entries 0, 1) and hi (entries 2, 3):
                // ls2 = 2 hi + 1 and ls1 - ls2 = 2 (lo - hi) as byte c & 3 of l2[c >> 2]
                // and (signed) of dl[c >> 2]; 128 + 2 lo - 2 hi never borrows.
                uint32_t l2[2], dl[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t w = h ? sc.y : sc.x;
                    const uint32_t hi2 = (w >> 3) & 0x1E1E1E1Eu, lo2 = (w << 1) & 0x1E1E1E1Eu;
                    l2[h] = hi2 | 0x01010101u;
                    dl[h] = ((lo2 | 0x80808080u) - hi2) ^ 0x80808080u;
                }
                int bi[4] = {0, 0, 0, 0};
                uint32_t u[4];
                xs_lane(o.q, u);
                uint4 g[8];
                uint2 m[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {   // all eight lookups in flight before the first use
                    const uint32_t w = u[c >> 1], code = (c & 1) ? w >> 16 : w;
                    g[c] = *reinterpret_cast<const uint4*>(lds + ((code & 0xff80u) | lo_x));
                    m[c] = *reinterpret_cast<const uint2*>(lds + perm(w, lo_s, (c & 1) ? 0x0C020600u : 0x0C020400u));
                }
                // sub-block c's two MFMAs are issued before sub-block c - 1's scale
                // multiply-adds read their results (no wait states between them)
                v4i C[8], C1[8];
#pragma unroll
                for (int c = 0; c <= 8; ++c) {
                    if (c < 8) {
                        const uint32_t* av = reinterpret_cast<const uint32_t*>(o.a) + 2 * c;
                        const long A = pack64(av[0], av[1]);
                        const uint32_t blo = bfi(m[c].x, g[c].z, g[c].x), bhi = bfi(m[c].y, g[c].w, g[c].y);
                        C[c] = mfma(A, pack64(blo, bhi), v4i{0, 0, 0, 0});
                        C1[c] = mfma(A, pack64(blo & mk, bhi & mk), v4i{0, 0, 0, 0});
                    }
                    if (c > 0) {
                        const int p = c - 1;
                        const int ls2 = int(__builtin_amdgcn_ubfe(l2[p >> 2], 8 * (p & 3), 8));
                        const int dls = __builtin_amdgcn_sbfe(int(dl[p >> 2]), 8 * (p & 3), 8);
#pragma unroll
                        for (int r = 0; r < RR; ++r) bi[r] = mad24(ls2, C[p][r], mad24(dls, C1[p][r], bi[r]));
                    }
                }
                if constexpr (TR) {
                    const int nbx = a.dim / 256;
                    const size_t rec = 2 * size_t(a.ff) * nbx + size_t(a.dim) * nb;
#pragma unroll
                    for (int r = 0; r < RR; ++r)
                        if (a.tint && po[r] >= 0)
                            a.tint[size_t(po[r]) * rec + 2 * size_t(a.ff) * nbx + size_t(row) * nb + size_t(b)] = bi[r];
                }
                const float ddf = h2f(reinterpret_cast<const uint16_t*>(lds + kL_RDD)[rl * nb + b]);
                const float4 hd4 = *reinterpret_cast<const float4*>(lds + kL_PD + 64 * b + 16 * e4);
                const float hd[4] = {hd4.x, hd4.y, hd4.z, hd4.w};
#pragma unroll
                for (int r = 0; r < RR; ++r) acc[r] = fmaf(__fmul_rn(ddf, hd[r]), float(bi[r]), acc[r]);
            };
            DnOps s0, s1;
            load(s0, 0);
            uint32_t t0 = touch(min(1, nb - 1)), t2 = touch(min(3, nb - 1));
            for (int b = 0; b < nb; b += 4) {
                load(s1, min(b + 1, nb - 1));
                sink(sunk, t0);
                t0 = touch(min(b + 5, nb - 1));
                __builtin_amdgcn_sched_barrier(0);   // the loads stay ahead of the compute
                compute(s0);
                load(s0, min(b + 2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 1 < nb) compute(s1);
                load(s1, min(b + 3, nb - 1));
                sink(sunk, t2);
                t2 = touch(min(b + 7, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 2 < nb) compute(s0);
                load(s0, min(b + 4, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (b + 3 < nb) compute(s1);
            }
            sink(sunk, t0 ^ t2);
#pragma unroll
            for (int r = 0; r < RR; ++r)
                if (po[r] >= 0) a.y[size_t(po[r]) * a.dim + row] = __fmul_rn(0.125f, acc[r]);
        };
        __syncthreads();   // the item's scales are staged
        if (wv * 16 >= rows) continue;   // wave-uniform: no rows of this wave in the last group
        if (tk.z <= 8) run.template operator()<2>();
        else if (tk.z <= 12) run.template operator()<3>();
        else run.template operator()<4>();
    }
    if (sunk == 0x9e3779b9u && lane == 64) a.y[0] = 0.0f;   // never true (lane < 64): keeps the touches
}

// ---------------------------------------------------------------------------
// Fixed-order combine per token (runtime.cpp:183-188): ascending expert id,
// out = fma(w, y, out) from +0, then + shared. A bad id contributes nothing.
// Wave 0 ranks the token's picks once (ascending id, equal ids in pick order:
// the stable order of an insertion sort) into LDS; every thread then issues
// its column's loads of all the token's rows before the fma chain.
// ---------------------------------------------------------------------------
// V values per thread (V = 4: 16-byte loads and stores; out and shared 16-byte
// aligned), each combined exactly as with V = 1.
template <int V>
__global__ __launch_bounds__(256) void gcombine_kernel(GroupArgs a) {
    __shared__ int s_row[16];     // pair row of rank r
    __shared__ float s_w[16];
    __shared__ int s_n;
    const int tok = blockIdx.y, t = threadIdx.x, k = a.k;
    if (t < 64) {
        const int id = t < k ? a.ids[size_t(tok) * k + t] : -1;
        const bool ok = t < k && id >= 0 && id < a.n_experts;
        int rank = 0;
        for (int j = 0; j < k; ++j) {
            const int idj = __shfl(id, j);
            const bool okj = idj >= 0 && idj < a.n_experts;
            rank += int(okj && (idj < id || (idj == id && j < t)));
        }
        if (ok) {
            s_row[rank] = tok * k + t;
            s_w[rank] = a.w[size_t(tok) * k + t];
        }
        const int n = __popcll(__ballot(ok));
        if (t == 0) s_n = n;
    }
    __syncthreads();
    const int c = (blockIdx.x * 256 + t) * V;
    if (c >= a.dim) return;   // dim is a multiple of 256
    const int n = s_n;
    using VT = std::conditional_t<V == 4, float4, float>;
    auto lanes = [](VT& x) -> float* { return reinterpret_cast<float*>(&x); };
    VT v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = r < n ? *reinterpret_cast<const VT*>(a.y + size_t(s_row[r]) * a.dim + c) : VT{};
    VT acc{};
#pragma unroll
    for (int r = 0; r < 16; ++r)
        if (r < n)
#pragma unroll
            for (int e = 0; e < V; ++e) lanes(acc)[e] = fmaf(s_w[r], lanes(v[r])[e], lanes(acc)[e]);
    if (a.shared) {
        VT sh = *reinterpret_cast<const VT*>(a.shared + size_t(tok) * a.dim + c);
#pragma unroll
        for (int e = 0; e < V; ++e) lanes(acc)[e] = __fadd_rn(lanes(acc)[e], lanes(sh)[e]);
    }
    *reinterpret_cast<VT*>(a.out + size_t(tok) * a.dim + c) = acc;
}

}  // namespace

hipError_t launch_grouped(const GroupArgs& args, int cus, hipStream_t s) {
    // gate/up: 12 waves per workgroup (3 per SIMD, 192 rows per item) where ff
    // allows, else 8; down: 12 (its last group of a task ragged)
    constexpr int NW = 8, NWD = 12;
    if (args.T < 1 || args.k < 1 || args.k > 16 || args.n_experts > kGroupMaxExperts || args.dim % (NW * 16) ||
        args.ff % (NW * 16) || args.dim % 256 || args.ff % 256 || args.dim > kGuNb * 256 || args.ff > kDnNb * 256)
        return hipErrorNotSupported;
    const bool gu12 = args.ff % (12 * 16) == 0;
    const int P = args.T * args.k;
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(1024), 0, s, args);
    const int nbx = args.dim / 256, nbh = args.ff / 256;
    if (args.tq8x || args.tq8h || args.th || args.tint) {   // the parity trace (separate instances)
        hipLaunchKernelGGL((q8k_rows_kernel<ROWS_X, true>), dim3((args.T * nbx + 3) / 4), dim3(256), 0, s, args.x,
                           args.T, nbx, args.xq, args.xd, args.pos, args.k, args.err, args.tq8x);
        if (gu12)
            hipLaunchKernelGGL((gu_kernel<12, true>), dim3(cus), dim3(12 * 64), 0, s, args);
        else
            hipLaunchKernelGGL((gu_kernel<NW, true>), dim3(cus), dim3(NW * 64), 0, s, args);
        hipLaunchKernelGGL((q8k_rows_kernel<ROWS_H, true>), dim3((P * nbh + 3) / 4), dim3(256), 0, s, args.h, P, nbh,
                           args.hq, args.hd, args.pos, args.k, args.err, args.tq8h);
        hipLaunchKernelGGL((dn_kernel<NWD, true>), dim3(cus), dim3(NWD * 64), 0, s, args);
    } else {
        hipLaunchKernelGGL((q8k_rows_kernel<ROWS_X, false>), dim3((args.T * nbx + 3) / 4), dim3(256), 0, s, args.x,
                           args.T, nbx, args.xq, args.xd, args.pos, args.k, args.err, nullptr);
        if (gu12)
            hipLaunchKernelGGL((gu_kernel<12, false>), dim3(cus), dim3(12 * 64), 0, s, args);
        else
            hipLaunchKernelGGL((gu_kernel<NW, false>), dim3(cus), dim3(NW * 64), 0, s, args);
        hipLaunchKernelGGL((q8k_rows_kernel<ROWS_H, false>), dim3((P * nbh + 3) / 4), dim3(256), 0, s, args.h, P, nbh,
                           args.hq, args.hd, args.pos, args.k, args.err, nullptr);
        hipLaunchKernelGGL((dn_kernel<NWD, false>), dim3(cus), dim3(NWD * 64), 0, s, args);
    }
    const bool al16 = (reinterpret_cast<uintptr_t>(args.out) | reinterpret_cast<uintptr_t>(args.shared)) % 16 == 0;
    if (al16) hipLaunchKernelGGL(gcombine_kernel<4>, dim3((args.dim / 4 + 255) / 256, args.T), dim3(256), 0, s, args);
    else hipLaunchKernelGGL(gcombine_kernel<1>, dim3((args.dim + 255) / 256, args.T), dim3(256), 0, s, args);
    return hipGetLastError();
}

}  // namespace xl::dev
