// fp8 x fp8 GEMM with per-token x per-output-channel dequantization and a
// fused bias / GELU(tanh) / AdaLN-gate epilogue, for gfx950 (MI355X).
//
//   v         = bf16(x_scale[m] * w_scale[n] * sum_k xq[m][k] wq[n][k])
//   v         = bf16(v + bias[n])                          (with a bias)
//   out[m][n] = bf16(epi(v))                               (none / GELU(tanh) / gate)
// rounding to bf16 where the reference's op sequence does (_scaled_mm with
// out_dtype=bf16, the bf16 bias add, then the epilogue on the bf16 tensor).
//
// Both operands are K-contiguous (xq [M, K], wq [N, K]), the "TN" layout of
// torch._scaled_mm(x_fp8, weight_fp8.t()) in the reference (fp8_linear.py:272).
//
// Main kernel (K % 256 == 0). A workgroup of 4 wavefronts computes a 256 (m) x
// 256 (n) output tile; each wave owns a 128 x 128 quadrant as 8 x 8
// v_mfma_f32_16x16x128_f8f6f4 tiles (256 fp32 accumulators per lane, in AGPRs).
// K advances in 128-byte blocks through two LDS stages (X and W tiles of 256
// rows x 128 bytes: 64 KiB a stage). Global -> LDS copies bypass VGPRs
// (buffer_load_dwordx4 ... lds) and move whole 128-byte rows -- half-line
// copies stream at two thirds of the rate on this part. A block is 64 MFMAs,
// each over the whole 128 K bytes: 8 groups, group j multiplying X fragment j by
// the wave's 8 W fragments. The W fragments sit in registers for the block, the
// next block's are read into a second set while this one's MFMAs run (so blocks
// come in pairs: K a multiple of 256), and the X fragments stream three groups
// ahead of their MFMAs. Two barriers per block free the W and X halves of a stage
// for the copies of block j+2. On random operand codes the 16 x 16 x 128
// instruction reaches 0.88 of the nominal peak in a bare loop where the
// 32 x 32 x 64 one reaches 0.75 (the part is power-limited and the smaller
// instruction draws less per FLOP).
// LDS rows are 128 bytes; the 16-byte chunk c of row r sits at c ^ s(r) (see
// row_swizzle: conflict-free for the 16-row fragment reads).
//
// MFMA orientation: the instruction's A operand is the W tile (its rows are
// output channels n) and its B operand the X tile (columns are tokens m), so
// each lane's accumulators come in runs of 4 consecutive n of one m: the
// epilogue stores 8 bytes (4 bf16) per lane.
//
// Tile order: workgroup b runs on XCD b % 8; tiles are renumbered so each XCD
// walks a contiguous run of the tile space, grouped kGroupM (4) m-tiles at a time,
// which keeps the X and W slices its 32 CUs share resident in that XCD's L2.
//
// K % 128 != 0 goes to a second kernel (BK = 128, 16x16x128 MFMA, two stages)
// whose last step is filled through VGPRs with zeros past K.
//
// The last round of tiles, when it would leave most compute units idle: rows of
// K >= 8192 split it along K (units storing binary32 partial sums to a
// workspace, then k_gemm_splitk_reduce); other shapes with at most a quarter of
// the units busy run it as 128 x 128 quadrants (k_gemm_fp8_quad, the same bits
// as whole tiles). A per-row gate and the residual apply in the fast epilogue's
// row layout (kEpiRowGate).
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "vdn_common.h"

namespace vdn {
namespace {

constexpr int BM = 256;        // tokens per tile
constexpr int BN = 256;        // output channels per tile
constexpr int kThreads = 256;  // 4 wavefronts, 2 (n) x 2 (m), 128 x 128 each
constexpr int kGroupM = 4;     // m-tiles per group of the tile order (GemmArgs::group_m)

typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;

// Internal epilogue (not an ABI value): VDN_FP8_EPI_GATE with a per-row gate index
// and/or a residual, on 16-byte rows -- the fast epilogue with the gate and the residual
// applied in the staging's row layout.
constexpr int kEpiRowGate = 4;

struct GemmArgs {
    const uint8_t* xq;
    const float* sx;
    const uint8_t* wq;
    const float* sw;
    int64_t M, N, K, ldx, ldw;
    const uint16_t* bias;
    const uint16_t* gate;
    const int32_t* gate_index;
    int64_t gate_rows, ldgate;
    const uint16_t* residual;
    int64_t ldres;
    uint16_t* out;
    int64_t ldo;
    int tiles_m, tiles_n;
    // K-block rotation: tile (tm, tn) walks its K blocks starting at block
    // ((tm + tn) % k_phase_mod) * k_phase_step (mod nk); 0 = no rotation.
    int k_phase_mod, k_phase_step;
    int group_m;   // m-tiles per group of the tile order
    // Split of the last partial round along K (long rows only): the first t_main tiles
    // (in tile order) run whole; each of the others runs as `splits` K slices, unit u
    // being slice u % splits of tile t_main + u / splits, whose fp32 partial sums go to
    // ws (65536 floats per unit, accumulator layout) and are summed by the reduction
    // kernel, slice by slice, before the epilogue. units = 0: no split (t_main = T).
    int t_main, splits, units;
    float* ws;
};

constexpr int64_t kUnitFloatsDev = 65536;   // floats of one split unit's partial sums (a 256 x 256 tile)

// Item v of a walk: whole tile v (v < t_main, all K blocks from the tile's rotated
// start), or split unit v - t_main (blocks [kb0, kb0 + cnt) of its tile, no rotation).
template <bool PARTIAL>
__device__ __forceinline__ void gemm_item(const GemmArgs& p, int nk, int v, int& tile, int& kb0, int& cnt, int& unit)
{
    if (!PARTIAL) {
        tile = v; kb0 = -1; cnt = nk; unit = -1;
    } else {
        // (integer division runs on the VALU: the results are made scalar again, as the
        // copies' inline assembly takes the block offset in an SGPR)
        unit = v - p.t_main;
        const int r = __builtin_amdgcn_readfirstlane(unit / p.splits);
        const int sl = unit - r * p.splits;
        tile = p.t_main + r;
        // (slice boundaries on even blocks: the K loop takes blocks two at a time)
        const int h = nk >> 1;
        kb0 = 2 * __builtin_amdgcn_readfirstlane(sl * h / p.splits);
        cnt = 2 * __builtin_amdgcn_readfirstlane((sl + 1) * h / p.splits) - kb0;
    }
}

// Renumbers workgroup b so that XCD (b % 8) gets a contiguous run of tiles,
// then maps the run index to (tile_m, tile_n) in groups of gm m-tiles.
__device__ __forceinline__ void tile_coords(int b, int tiles_m, int tiles_n, int gm, int& tm, int& tn)
{
    const int T = tiles_m * tiles_n;
    const int q = T / 8, r = T % 8, xcd = b % 8, local = b / 8;
    const int t = (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
    const int group = gm * tiles_n;
    const int first_m = (t / group) * gm;
    const int gsize = min(tiles_m - first_m, gm);
    tm = first_m + (t % group) % gsize;
    tn = (t % group) / gsize;
}

// Epilogue for 4 consecutive output channels n .. n+3 of token m: the
// reference's rounding points; returns the 4 bf16 results packed.
template <int EPI>
__device__ __forceinline__ uint2 epi4(const GemmArgs& p, int64_t m, int64_t n, const float* acc, float sxm,
                                      const uint16_t* grow)
{
    const float4 sw = *reinterpret_cast<const float4*>(p.sw + n);
    const float swv[4] = {sw.x, sw.y, sw.z, sw.w};
    float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.bias) {
        const uint2 b = *reinterpret_cast<const uint2*>(p.bias + n);
        bv[0] = bf16_lo(b.x); bv[1] = bf16_hi(b.x); bv[2] = bf16_lo(b.y); bv[3] = bf16_hi(b.y);
    }
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[e] = round_bf16(acc[e] * (sxm * swv[e]));
        if (p.bias) v[e] = round_bf16(v[e] + bv[e]);
    }
    if (EPI == VDN_FP8_EPI_GELU_TANH) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
    } else if (EPI == VDN_FP8_EPI_GATE) {
        const uint2 gv = *reinterpret_cast<const uint2*>(grow + n);
        v[0] *= bf16_lo(gv.x); v[1] *= bf16_hi(gv.x); v[2] *= bf16_lo(gv.y); v[3] *= bf16_hi(gv.y);
        if (p.residual) {
            const uint2 rv = *reinterpret_cast<const uint2*>(p.residual + m * p.ldres + n);
            v[0] += bf16_lo(rv.x); v[1] += bf16_hi(rv.x); v[2] += bf16_lo(rv.y); v[3] += bf16_hi(rv.y);
        }
    }
    return make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

template <int EPI>
__device__ __forceinline__ void store4(const GemmArgs& p, int64_t m, int64_t n, const float* acc, float sxm,
                                       const uint16_t* grow)
{
    if constexpr (EPI == VDN_FP8_EPI_F32) {   // binary32 x_scale * w_scale * acc, as tile_epilogue's
        const float4 sw = *reinterpret_cast<const float4*>(p.sw + n);
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + m * p.ldo + n) =
            make_float4(acc[0] * (sxm * sw.x), acc[1] * (sxm * sw.y), acc[2] * (sxm * sw.z), acc[3] * (sxm * sw.w));
    } else {
        *reinterpret_cast<uint2*>(p.out + m * p.ldo + n) = epi4<EPI>(p, m, n, acc, sxm, grow);
    }
}

template <int EPI>
__device__ __forceinline__ const uint16_t* gate_row(const GemmArgs& p, int64_t m)
{
    if (EPI != VDN_FP8_EPI_GATE) return nullptr;
    const int64_t gi = p.gate_index ? min(max((int64_t)p.gate_index[m], (int64_t)0), p.gate_rows - 1) : 0;
    return p.gate + gi * p.ldgate;
}

// Buffer descriptor (raw, 32-bit data format, gfx9 family) over the valid rows
// of a tile: rows past M (or N) read as zeros. Wave-uniform, so in SGPRs.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint8_t* base, int64_t rows, int64_t ld)
{
    const int64_t bytes = min(rows, (int64_t)256) * ld;
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)min(bytes, (int64_t)0x7fffffff), kRsrcWord3);
}

// One wave-wide 16-byte-per-lane copy global -> LDS: lane L's 16 bytes at
// buffer offset voff + soff land at LDS byte lds + 16 L. Written as inline
// assembly so that the compiler does not treat every later LDS read as
// dependent on it (it would wait for all such copies, serializing the
// pipeline); the kernel waits on vmcnt itself. M0 carries the LDS address and
// is restored afterwards; s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void copy16_to_lds(i32x4_t rsrc, uint32_t lds, uint32_t voff, uint32_t soff)
{
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
        : "memory");
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14)
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | (0 << 8) | ((vm >> 4) << 14); }

// This wave's copies, except the VM most recent, have landed and its LDS reads
// are done; then all waves meet. The scheduling barriers keep the compiler from
// moving instructions across (MFMAs touch no memory and would otherwise float).
template <int VM>
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(VM));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// As wave_sync, without waiting for this wave's LDS reads.
template <int VM>
__device__ __forceinline__ void wave_sync_vm()
{
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------
// main kernel: K % 128 == 0, persistent
// ---------------------------------------------------------------------------
// Row r, 16-byte chunk c (0..7) of a 128-byte-row LDS tile sits at chunk c ^ s(r),
// s(r) = bits 1, 0, 2 of r. A 16 x 128-byte fragment read (lane L: row L % 16, chunk
// 2 (L / 16), then the next chunk) runs without bank conflicts under this swizzle --
// measured over every XOR swizzle of the row's low four bits: 1342 of the 4096 run at
// the full rate, the XOR with bits 1..3 of the row (conflict-free for the 32-row reads
// of the 32 x 32 x 64 instruction) at half of it.
__device__ __forceinline__ int row_swizzle(int row) { return ((row >> 1) & 1) | ((row & 1) << 1) | (row & 4); }

namespace mainloop {
constexpr int BK = 128;                     // K bytes per block (one LDS stage)
constexpr int kStage = (BM + BN) * BK;      // 64 KiB: X tile, then W tile
constexpr int kCopies = BM * BK / 1024 / 4; // 1 KiB copies per wave per tile per block (8)
constexpr int kBlockCopies = 2 * kCopies;   // X and W: 16 per wave per block
constexpr int kScal = 2 * kStage;           // per-tile vectors, two buffers of 4 x 1 KiB
constexpr int kStgRow = 144;                // epilogue staging row: 128 bytes + 16 of padding
constexpr int kStgWave = 32 * kStgRow;      // 32 rows per wave
constexpr int kStg = kScal + 8192;          // epilogue staging
constexpr int kLds = kStg + 4 * kStgWave;   // 154 KiB
constexpr int kEpiStores = 32;              // 16-byte stores per wave per tile (fast epilogue)
constexpr int kStoreNT = 2;                 // cache policy of the output stores: non-temporal (the
                                            // output streams; keeps L2 for the operand panels)

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * BK + ((chunk ^ row_swizzle(row)) << 4); }
}  // namespace mainloop

__device__ __forceinline__ i32x4_t rsrc_words(const void* base, int64_t bytes)
{
    const uint64_t a = (uint64_t)base;
    bytes = max(min(bytes, (int64_t)0x7fffffff), (int64_t)0);
    return i32x4_t{__builtin_amdgcn_readfirstlane((int)(a & 0xffffffffu)),
                   __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffffu)),
                   __builtin_amdgcn_readfirstlane((int)bytes), kRsrcWord3};
}

// Epilogue of the tile at (m0, n0) with its vectors in scalar buffer sb of smem
// acc[i][j][e] is n = wn*128 + 16 i + 4 (lane/16) + e, m = wm*128 + 16 j +
// lane%16 (tile-relative). Per 32-row band u and per 64-column half th the wave
// finishes its 32 x 64 slab (accumulators i = 4 th .. 4 th + 3, j = 2 u, 2 u + 1)
// in that layout (4 consecutive n per lane),
// writes it to its staging (32 rows of 128 bytes, padded to 144), reads it
// back by rows and stores 16-byte pieces of whole 128-byte row segments: lane
// L covers row 8 i + L/8, channels 8 (L%8) .. +7. The gate and residual
// apply in that row layout.
// The epilogue's slabs in order: sidx = 4 (1 - th) + 3 - u, (th, u) = (1, 3), (1, 2), ..
// (0, 0). A slab mask (bit sidx; -1: every slab) restricts an epilogue to some of them.
constexpr bool slab_in(int mask, int s) { return mask < 0 || ((mask >> s) & 1); }
constexpr int slab_first(int mask) { return mask < 0 ? 0 : __builtin_ctz((unsigned)mask); }
constexpr int slab_last(int mask) { return mask < 0 ? 7 : 31 - __builtin_clz((unsigned)mask); }

// scal: the tile's vectors (4 KiB: w_scale, x_scale, bias, gate index or gate row, 1 KiB
// each); stg: this wave's staging rows. Shared by the main kernel, the split-K reduction
// (four waves on a quadrant, each its 32 rows) and the quadrant kernel (each wave 64 x
// 64): MASK >= 0 restricts the epilogue to those slabs (bit sidx).
template <int EPI, bool FAST, int MASK = -1>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& p, const uint8_t* scal, uint8_t* stg,
                                              f32x4_t (&acc)[8][8], int64_t m0, int64_t n0, int wave)
{
    using namespace mainloop;
    const int wn = wave & 1, wm = wave >> 1;
    if constexpr (EPI == VDN_FP8_EPI_F32) {
        // binary32 output x_scale * w_scale * acc, stored from the accumulators: 16 bytes
        // (4 consecutive n of one m) per accumulator and lane; N % 4 == 0 keeps n .. n + 3
        // inside a row whenever n is
        uint32_t zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        const int el = (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) + zero);
        const int fr = el & 15, fg = el >> 4;
        const float* s_sw = reinterpret_cast<const float*>(scal);
        const float* s_sx = reinterpret_cast<const float*>(scal + 1024);
        float* out = reinterpret_cast<float*>(p.out);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int ml = wm * 128 + 16 * j + fr;
            const int64_t m = m0 + ml;
            const float sxm = s_sx[ml];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (!slab_in(MASK, 4 * (1 - (i >> 2)) + 3 - (j >> 1))) continue;
                const int nl = wn * 128 + 16 * i + 4 * fg;
                const int64_t n = n0 + nl;
                const float4 sw = *reinterpret_cast<const float4*>(s_sw + nl);
                if (m < p.M && n < p.N)
                    *reinterpret_cast<float4*>(out + m * p.ldo + n) =
                        make_float4(acc[i][j][0] * (sxm * sw.x), acc[i][j][1] * (sxm * sw.y),
                                    acc[i][j][2] * (sxm * sw.z), acc[i][j][3] * (sxm * sw.w));
                acc[i][j] = f32x4_t{};   // the next tile starts from zero
            }
        }
        (void)stg;
        return;
    }
    const bool gate16 = ((p.ldgate & 7) == 0) && (((uintptr_t)p.gate & 15) == 0);
    const bool res16 = ((p.ldres & 7) == 0) && (((uintptr_t)p.residual & 15) == 0);
    // Every lane-dependent value here derives from an opaque zero, so the
    // compiler recomputes it per tile instead of holding it in registers
    // across the K loop.
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    const int el = (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) + zero);
    const int fr = el & 15, fg = el >> 4, cc = el & 7, rl = el >> 3;
    const float* s_sw = reinterpret_cast<const float*>(scal);
    const float* s_sx = reinterpret_cast<const float*>(scal + 1024);
    const uint16_t* s_bias = reinterpret_cast<const uint16_t*>(scal + 2048);
    const int32_t* s_gi = reinterpret_cast<const int32_t*>(scal + 3072);
    const uint16_t* s_gate = reinterpret_cast<const uint16_t*>(scal + 3072);
    const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.out + m0 * p.ldo), 0, (int)min(min(p.M - m0, (int64_t)BM) * p.ldo * 2, (int64_t)0x7fffffff), kRsrcWord3);
    const uint32_t ldo2 = (uint32_t)p.ldo * 2;
    // Slabs in order (th, u) = (1, 3), (1, 2), .. (0, 0). A column half's per-column
    // vectors (w_scale, bias and a broadcast gate row, unpacked to binary32) are read
    // from LDS once and held in registers across its four slabs -- the K loop's
    // fragment registers are free here. On the fast path the stores trail by one
    // slab: the previous slab's rows are read back from the staging before this
    // slab's values overwrite it (a wave's LDS operations run in order), so its
    // computation hides that read's latency.
    const bool has_bias = p.bias != nullptr;
    float hsw[4][4], hb[4][4], hg[4][4];
    auto hoist = [&](int th) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int nl = wn * 128 + 64 * th + 16 * ii + 4 * fg;
            const float4 sw = *reinterpret_cast<const float4*>(s_sw + nl);
            hsw[ii][0] = sw.x; hsw[ii][1] = sw.y; hsw[ii][2] = sw.z; hsw[ii][3] = sw.w;
            if (has_bias) {
                const uint2 b = *reinterpret_cast<const uint2*>(s_bias + nl);
                hb[ii][0] = bf16_lo(b.x); hb[ii][1] = bf16_hi(b.x);
                hb[ii][2] = bf16_lo(b.y); hb[ii][3] = bf16_hi(b.y);
            }
            if (EPI == VDN_FP8_EPI_GATE && FAST) {
                const uint2 gv = *reinterpret_cast<const uint2*>(s_gate + nl);
                hg[ii][0] = bf16_lo(gv.x); hg[ii][1] = bf16_hi(gv.x);
                hg[ii][2] = bf16_lo(gv.y); hg[ii][3] = bf16_hi(gv.y);
            }
        }
    };
    // bf16 GEMM output, then the bf16 bias add: each rounding done two values per
    // conversion, the second one's pairs being the stored words (opaque, so the
    // compiler keeps the pairs); one uniform branch per slab
    auto compute = [&](int th, int u, auto with_bias) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const float sxm = s_sx[wm * 128 + 32 * u + 16 * jj + fr];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const float* sw = hsw[ii];
                // A rounding to bf16 that the bias add or GELU reads is one conversion per
                // value (round_bf16_hi: no unpacking); the last one converts the stored
                // pairs. The gate kernels keep the packed pairs and unpack them (one value
                // per conversion there made the compiler spill).
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[4 * th + ii][2 * u + jj][e] * (sxm * sw[e]);
                uint32_t r01, r23;
                if (EPI != VDN_FP8_EPI_GATE) {
                    if (decltype(with_bias)::value) {
                        const float* bb = hb[ii];
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = round_bf16_hi(v[e]) + bb[e];
                    }
                    if (EPI == VDN_FP8_EPI_GELU_TANH) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(round_bf16_hi(v[e]));   // of the bf16 output
                    }
                    r01 = pack_bf16x2(v[0], v[1]);
                    r23 = pack_bf16x2(v[2], v[3]);
                    asm volatile("" : "+v"(r01), "+v"(r23));
                } else {
                    r01 = pack_bf16x2(v[0], v[1]);
                    r23 = pack_bf16x2(v[2], v[3]);
                    asm volatile("" : "+v"(r01), "+v"(r23));
                    if (decltype(with_bias)::value) {
                        const float* bb = hb[ii];
                        r01 = pack_bf16x2(bf16_lo(r01) + bb[0], bf16_hi(r01) + bb[1]);
                        r23 = pack_bf16x2(bf16_lo(r23) + bb[2], bf16_hi(r23) + bb[3]);
                        asm volatile("" : "+v"(r01), "+v"(r23));
                    }
                    if (FAST) {   // broadcast gate row, no residual
                        const float* gg = hg[ii];
                        r01 = pack_bf16x2(bf16_lo(r01) * gg[0], bf16_hi(r01) * gg[1]);
                        r23 = pack_bf16x2(bf16_lo(r23) * gg[2], bf16_hi(r23) * gg[3]);
                    }
                }
                *reinterpret_cast<uint2*>(stg + (16 * jj + fr) * kStgRow + 32 * ii + 8 * fg) = make_uint2(r01, r23);
            }
        }
        // these accumulators start the next tile from zero
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            acc[4 * th + ii][2 * u] = f32x4_t{};
            acc[4 * th + ii][2 * u + 1] = f32x4_t{};
        }
    };
    // fast path: the slab's rows 8 i + L/8 from the staging, then their stores (byte
    // offset of the row, or out of range past N)
    uint4 pv[4];
    auto read_slab = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = *reinterpret_cast<const uint4*>(stg + (8 * i + rl) * kStgRow + (cc << 4));
    };
    // (the four offsets first, then the four stores back to back and their wait states)
    // Row gate: the gate table row gate_index[m] and the residual for the slab's rows
    // 8 i + L/8, columns 8 (L % 8) .. + 7 of the column half, by 16-byte buffer loads
    // issued two slabs ahead of their use into one of two register sets (rows past M and
    // columns past N read outside the descriptors: zeros), then, in the stores' row
    // layout, out = bf16(residual + gate * v) -- the gated residual kernel's arithmetic.
    constexpr bool kRowGate = EPI == kEpiRowGate;
    const bool has_res = p.residual != nullptr;
    const int64_t rows_here = min(p.M - m0, (int64_t)BM);
    const __amdgpu_buffer_rsrc_t rsr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kRowGate && has_res ? p.residual + m0 * p.ldres : nullptr), 0,
        kRowGate && has_res ? (int)(((rows_here - 1) * p.ldres + p.N) * 2) : 0, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t gsr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kRowGate ? p.gate : nullptr), 0, kRowGate ? (int)(((p.gate_rows - 1) * p.ldgate + p.N) * 2) : 0,
        kRsrcWord3);
    uint4 rres[2][4], rgat[2][4];
    auto load_rows = [&](int th, int u, int set) {
        const int64_t n = n0 + wn * 128 + 64 * th + 8 * cc;
        const bool nin = n < p.N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ml = wm * 128 + 32 * u + 8 * i + rl;
            const int64_t gi = min(max((int64_t)s_gi[ml], (int64_t)0), p.gate_rows - 1);
            const uint32_t ro = nin ? (uint32_t)(((int64_t)ml * p.ldres + n) * 2) : 0x80000000u;
            const uint32_t go = nin ? (uint32_t)((gi * p.ldgate + n) * 2) : 0x80000000u;
            rres[set][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsr, ro, 0, kBufferLoadOnce));
            rgat[set][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(gsr, go, 0, 0));
        }
    };
    auto apply_rows = [&](int set) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t vw[4] = {pv[i].x, pv[i].y, pv[i].z, pv[i].w};
            const uint32_t gw[4] = {rgat[set][i].x, rgat[set][i].y, rgat[set][i].z, rgat[set][i].w};
            const uint32_t rw[4] = {rres[set][i].x, rres[set][i].y, rres[set][i].z, rres[set][i].w};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // without a residual the product is stored as it is (no + 0: -0 stays -0)
                float lo = bf16_lo(gw[e]) * bf16_lo(vw[e]);
                float hi = bf16_hi(gw[e]) * bf16_hi(vw[e]);
                if (has_res) { lo = bf16_lo(rw[e]) + lo; hi = bf16_hi(rw[e]) + hi; }
                o[e] = pack_bf16x2(lo, hi);
            }
            pv[i] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    };
    auto store_slab = [&](int th, int u, int set) {
        if constexpr (kRowGate) apply_rows(set);
        const int64_t n = n0 + wn * 128 + 64 * th + 8 * cc;
        const uint32_t off0 = (uint32_t)(wm * 128 + 32 * u + rl) * ldo2 + (uint32_t)(n * 2);
        uint32_t off[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) off[i] = n < p.N ? off0 + (uint32_t)(8 * i) * ldo2 : 0x80000000u;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, pv[i]), orr, off[i], 0, kStoreNT);
        settle_stores();
    };
    // (MASK >= 0: two slabs, kFirst and kLast)
    static_assert(MASK < 0 || __builtin_popcount((unsigned)MASK) == 2, "a slab mask holds two slabs");
    constexpr int kFirst = slab_first(MASK), kLast = slab_last(MASK);
    constexpr int kStep = MASK < 0 ? 1 : kLast - kFirst;
    // (the register set of slab sidx: the parity of its place in the order)
    auto set_of = [](int sidx) { return ((sidx - kFirst) / kStep) & 1; };
    if constexpr (kRowGate) load_rows(1 - kFirst / 4, 3 - kFirst % 4, 0);
#pragma unroll
    for (int sidx = 0; sidx < 8; ++sidx) {
        const int th = 1 - sidx / 4, u = 3 - sidx % 4;
        if (MASK >= 0 && !((MASK >> sidx) & 1)) continue;
        if (MASK >= 0 || sidx % 4 == 0) hoist(th);
        if (FAST && sidx > kFirst) read_slab();   // the previous slab, before this one overwrites it
        if (has_bias) compute(th, u, std::true_type{});
        else compute(th, u, std::false_type{});
        if (FAST) {
            if (sidx > kFirst) store_slab(1 - (sidx - kStep) / 4, 3 - (sidx - kStep) % 4, set_of(sidx - kStep));
            if constexpr (kRowGate) {
                if (sidx < kLast) load_rows(1 - (sidx + kStep) / 4, 3 - (sidx + kStep) % 4, set_of(sidx + kStep));
            }
        } else {
            const int64_t n = n0 + wn * 128 + 64 * th + 8 * cc;
            const bool full = n + 8 <= p.N;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 8 * i + rl;
                uint4 v = *reinterpret_cast<const uint4*>(stg + r * kStgRow + (cc << 4));
                const int ml = wm * 128 + 32 * u + r;
                const int64_t m = m0 + ml;
                if (m >= p.M || n >= p.N) continue;
                if (EPI == VDN_FP8_EPI_GATE) {
                    const int64_t gi = p.gate_index ? min(max((int64_t)s_gi[ml], (int64_t)0), p.gate_rows - 1) : 0;
                    const uint16_t* gp = p.gate + gi * p.ldgate + n;
                    uint4 g;
                    if (gate16 && full) g = *reinterpret_cast<const uint4*>(gp);
                    else {
                        const uint2 g0 = *reinterpret_cast<const uint2*>(gp);
                        const uint2 g1 = full ? *reinterpret_cast<const uint2*>(gp + 4) : make_uint2(0u, 0u);
                        g = make_uint4(g0.x, g0.y, g1.x, g1.y);
                    }
                    uint4 rv = make_uint4(0u, 0u, 0u, 0u);
                    if (p.residual) {
                        const uint16_t* rp = p.residual + m * p.ldres + n;
                        if (res16 && full) rv = *reinterpret_cast<const uint4*>(rp);
                        else {
                            const uint2 r0 = *reinterpret_cast<const uint2*>(rp);
                            const uint2 r1 = full ? *reinterpret_cast<const uint2*>(rp + 4) : make_uint2(0u, 0u);
                            rv = make_uint4(r0.x, r0.y, r1.x, r1.y);
                        }
                    }
                    const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, gw[4] = {g.x, g.y, g.z, g.w},
                                   rw[4] = {rv.x, rv.y, rv.z, rv.w};
                    uint32_t o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float lo = bf16_lo(vw[e]) * bf16_lo(gw[e]), hi = bf16_hi(vw[e]) * bf16_hi(gw[e]);
                        if (p.residual) { lo += bf16_lo(rw[e]); hi += bf16_hi(rw[e]); }
                        o[e] = pack_bf16x2(lo, hi);
                    }
                    v = make_uint4(o[0], o[1], o[2], o[3]);
                }
                uint16_t* dst = p.out + m * p.ldo + n;
                *reinterpret_cast<uint2*>(dst) = make_uint2(v.x, v.y);
                if (full) *reinterpret_cast<uint2*>(dst + 4) = make_uint2(v.z, v.w);
            }
        }
        // one slab at a time: unbounded interleaving of slabs runs out of VGPRs
        __builtin_amdgcn_sched_barrier(0);
    }
    if (FAST) {   // the last slab
        read_slab();
        store_slab(1 - kLast / 4, 3 - kLast % 4, set_of(kLast));
    }
}

// One workgroup per CU walks tiles blockIdx.x, + gridDim.x, ... The copies form
// one stream of 128-byte K blocks across those tiles, so the next tile's first
// two blocks are in flight while this tile's epilogue runs. The block schedule
// (8 groups of 8 MFMAs, two barriers) is described at the K loop below.
// A tile's vectors (w_scale, x_scale, bias, gate rows) are copied into one of
// two scalar buffers at the start of the tile before, one copy per wave. The
// epilogue stages through LDS of its own.
//
// FAST (16-byte aligned output rows; a broadcast gate row travels with the tile's
// vectors, a per-row gate and the residual -- kEpiRowGate -- are loaded by the
// epilogue two slabs ahead of their use): the epilogue issues exactly kEpiStores
// buffer stores per wave, columns past N sent out of range (dropped), and every
// load it issues has landed when it ends, so the waits that follow count the
// stores (conservatively, the counter retiring in issue order) and the stores
// drain while the next tile runs. Otherwise the waits also cover the epilogue's
// memory operations.
// PARTIAL: the split units instead of the whole tiles (one per workgroup, its K slice,
// the partial sums stored raw; a launch of its own, so that the whole-tile kernel keeps
// one straight-line epilogue; EPI and FAST do not matter to it: one instance serves).
template <int EPI, bool FAST, bool PARTIAL>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemm_fp8(GemmArgs p)
{
    using namespace mainloop;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];
    constexpr int kE = FAST ? kEpiStores : 0;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int nk = (int)(p.K / BK);
    const int stride = gridDim.x;
    const int v_begin = PARTIAL ? p.t_main : 0;
    const int n_items = PARTIAL ? p.t_main + p.units : p.t_main;

    // Copies: this wave fills rows 64 wave .. 64 wave + 63 of each tile, 8 rows
    // (1 KiB) per copy. Lane L lands at row +L/8, physical chunk L%8, so it
    // fetches logical chunk (L%8) ^ row_swizzle(row), row = 64 wave + 8 i + L/8.
    // (recomputed per tile from an opaque lane index, with every other lane-dependent
    // value of the K loop, so that none is held in registers across the epilogue)
    uint32_t xoff[kCopies], woff[kCopies];
    auto opaque_lane = [&]() -> int {
        uint32_t zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        return (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) + zero);
    };
    auto copy_offsets = [&](int l) {
#pragma unroll
        for (int i = 0; i < kCopies; ++i) {
            const int r = 64 * wave + 8 * i + (l >> 3);
            const int c = (l & 7) ^ row_swizzle(r);
            xoff[i] = (uint32_t)(r * p.ldx) + c * 16;
            woff[i] = (uint32_t)(r * p.ldw) + c * 16;
        }
    };
    copy_offsets(lane);
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void_t*)smem;

    // Producer: the next block to copy is block pj of item pv (pnk blocks from block
    // pphase, wrapping). Blocks of items past the end still issue their copies, through
    // empty descriptors (zeros, no memory read), so the vmcnt bookkeeping stays fixed.
    int pv = v_begin + blockIdx.x, pj = 0, pphase = 0, pkb = 0, pnk = nk;
    i32x4_t xr, wr;
    auto producer_tile = [&]() {
        int64_t xb = 0, wb = 0;
        const uint8_t* xa = p.xq;
        const uint8_t* wa = p.wq;
        pphase = 0;
        pnk = nk;
        if (pv < n_items) {
            int tile, kb0, unit, tm, tn;
            gemm_item<PARTIAL>(p, nk, pv, tile, kb0, pnk, unit);
            tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
            if (kb0 >= 0) pphase = kb0;
            else if (p.k_phase_mod > 0) pphase = (((tm + tn) % p.k_phase_mod) * p.k_phase_step) % nk;
            const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
            xa += m0 * p.ldx;
            wa += n0 * p.ldw;
            xb = min(p.M - m0, (int64_t)BM) * p.ldx;
            wb = min(p.N - n0, (int64_t)BN) * p.ldw;
        }
        xr = rsrc_words(xa, xb);
        wr = rsrc_words(wa, wb);
        pkb = pphase * BK;
        asm volatile("s_nop 4");   // SGPR write by VALU -> use as a buffer descriptor
    };
    // Copy c (0..15) of the producer's block into stage st: c < 8 is X rows
    // 64 wave + 8 c .., else W rows.
    auto copy = [&](int st, int c) {
        const uint32_t dst = lds_base + (uint32_t)st * kStage;
        const uint32_t kb = (uint32_t)pkb;
        const int i = c & 7;
        if (c < 8) copy16_to_lds(xr, dst + (64 * wave + 8 * i) * BK, xoff[i], kb);
        else copy16_to_lds(wr, dst + BM * BK + (64 * wave + 8 * i) * BK, woff[i], kb);
    };
    auto advance = [&]() {
        if (++pj == pnk) {
            pj = 0;
            pv += stride;
            producer_tile();
        } else {
            const int kbi = pj + pphase;
            pkb = (kbi >= nk ? kbi - nk : kbi) * BK;
        }
    };
    // The vectors of the k-th tile of this workgroup go to scalar buffer k % 2:
    // wave 0 w_scale[n0 ..+255], wave 1 x_scale[m0 ..+255], wave 2 bias[n0 ..+511]
    // (256 used), wave 3 gate_index[m0 ..+255] -- or, for a broadcast gate on the
    // fast path, the gate row gate[0][n0 ..+511]. Missing ones read as zeros.
    auto scal_copy = [&](int t, int buf) {
        const void* base = p.sx;
        int64_t bytes = 0;
        if (t < p.t_main) {   // whole tiles only (split units store raw partial sums)
            int tm, tn;
            tile_coords(t, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
            const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
            if (wave == 0) { base = p.sw + n0; bytes = min(p.N - n0, (int64_t)256) * 4; }
            else if (wave == 1) { base = p.sx + m0; bytes = min(p.M - m0, (int64_t)256) * 4; }
            else if (wave == 2) { if (p.bias) { base = p.bias + n0; bytes = min(p.N - n0, (int64_t)512) * 2; } }
            else if (EPI == VDN_FP8_EPI_GATE && FAST) { base = p.gate + n0; bytes = min(p.N - n0, (int64_t)512) * 2; }
            else if (p.gate_index) { base = p.gate_index + m0; bytes = min(p.M - m0, (int64_t)256) * 4; }
        }
        const i32x4_t r = rsrc_words(base, bytes);
        asm volatile("s_nop 4");
        // the lane index recomputed here rather than kept live across the K loop
        uint32_t zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        const uint32_t l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) + zero;
        copy16_to_lds(r, lds_base + kScal + buf * 4096 + wave * 1024, l * 16, 0);
    };

    // acc[i][j] += W fragment i x X fragment j: 16 (n) x 16 (m) outputs over the whole block
    f32x4_t acc[8][8];
    auto fence = [&]() { __builtin_amdgcn_sched_barrier(0); };

    auto epilogue = [&](int64_t m0, int64_t n0, int sb) {
        tile_epilogue<EPI, FAST>(p, smem + kScal + sb * 4096, smem + kStg + wave * kStgWave, acc, m0, n0, wave);
    };

    // Prologue: the first tile's vectors, then blocks 0 and 1 of the stream.
    producer_tile();
    scal_copy(v_begin + blockIdx.x, 0);
    // W copies (c = 8..15) before X copies (c = 0..7), as in the loop
#pragma unroll
    for (int c = 0; c < kBlockCopies; ++c) copy(0, (c + kCopies) % kBlockCopies);
    advance();
#pragma unroll
    for (int c = 0; c < kBlockCopies; ++c) copy(1, (c + kCopies) % kBlockCopies);
    advance();

#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{};   // the epilogue re-zeroes them per tile
    int g = 0;    // stream index of the block being computed
    int k = 0;    // tiles done by this workgroup

    for (int v = v_begin + blockIdx.x; v < n_items; v += stride, ++k) {
        int tile, kb0, cnt, unit, tm, tn;
        gemm_item<PARTIAL>(p, nk, v, tile, kb0, cnt, unit);
        // (opaque: conditions on it are then evaluated per block, not hoisted out of
        // the tile loop into registers held across the epilogue)
        asm volatile("" : "+s"(cnt));
        tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
        // Block g has landed once only block g+1's copies -- and, after the first
        // tile, the previous epilogue's stores -- may be pending.
        if (k == 0) wave_sync<kBlockCopies>();
        else wave_sync<kBlockCopies + kE>();
        scal_copy(v + stride, (k + 1) & 1);   // every wave is past the epilogue that used that buffer
        const int el = opaque_lane();
        copy_offsets(el);
        // Fragments of the block in stage st: 16 rows x 128 K bytes; lane L reads row
        // (base + L % 16), k bytes 32 (L / 16) .. +31, as two 16-byte chunks. W fragment
        // i is W rows wn*128 + 16 i .., X fragment j is X rows wm*128 + 16 j ..
        const int fr = el & 15, fg = el >> 4;
        auto read_frag = [&](const uint8_t* s, int row) -> i32x8_t {
            const uint4 lo = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg));
            const uint4 hi = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg + 1));
            return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        };
        auto read_w = [&](int st, int i) { return read_frag(smem + st * kStage + BM * BK, wn * 128 + 16 * i + fr); };
        auto read_x = [&](int st, int j) { return read_frag(smem + st * kStage, wm * 128 + 16 * j + fr); };
        // W fragments of the block being computed and of the next one (read into the
        // other set while this block's MFMAs run); X fragments four at a time, in rotation.
        // (Declared per tile: nothing of them lives across the epilogue.)
        i32x8_t wa[8], wb[8], xf[4];
        // Block g (j-th of the tile's cnt blocks, stage st = g % 2): 8 groups of 8 MFMAs,
        // group jx multiplying X fragment jx by the 8 W fragments.
        //   start (P0): W copies of block g+1 have landed in every wave, and every wave
        //     is done reading block g's W fragments (read during block g-1, or at the
        //     tile's start); group 1 then issues the W copies of block g+2 into stage st.
        //   group jx reads X fragment jx+3 (groups 5-7: block g+1's X fragments 0-2), three
        //     groups ahead of its MFMAs (one group ahead left them waiting on the read), and
        //     W fragment jx of block g+1.
        //   group 5 (P5): X copies of block g+1 have landed, every wave is done with block
        //     g's X fragments (the last read in group 4); groups 5 and 6 issue the X copies
        //     of block g+2 into stage st.
        // Copies newer than the awaited ones at P0 and P5: 8, plus in a tile's first block
        // the previous epilogue's stores and the vector copy. The tile's last block reads
        // the next one's fragments too (those of the next tile's first block, which the
        // next tile reads again): one code path, so the compiler's LDS waits count only
        // what each MFMA needs.
        // odd: which W set is current (wa in even blocks).
        auto kblock = [&](auto odd, int j) {
            i32x8_t (&wc)[8] = decltype(odd)::value ? wb : wa;
            i32x8_t (&wx)[8] = decltype(odd)::value ? wa : wb;
            const int st = g & 1;
            auto sync = [&]() {
                if (j > 0) wave_sync<kCopies>();
                else if (k > 0) wave_sync<kCopies + 1 + kE>();
                else wave_sync<kCopies + 1>();
            };
            sync();
    #pragma unroll
            for (int jx = 0; jx < 8; ++jx) {
                if (jx == 5) sync();
    #pragma unroll
                for (int i = 0; i < 8; ++i) {
                    acc[i][jx] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wc[i], xf[jx & 3], acc[i][jx],
                                                                                   0, 0, 0, 0, 0, 0);
                    fence();
                    if (i == 0) xf[(jx + 3) & 3] = jx < 5 ? read_x(st, jx + 3) : read_x(st ^ 1, jx - 5);
                    if (i == 4) wx[jx] = read_w(st ^ 1, jx);
                    if (jx >= 1 && jx <= 4 && (i == 2 || i == 6)) copy(st, kCopies + 2 * (jx - 1) + (i == 6));   // W copies of block g+2
                    if ((jx == 5 || jx == 6) && (i & 1)) copy(st, 4 * (jx - 5) + (i >> 1));   // X copies of block g+2
                    if (jx == 6 && i == 7) advance();
                    fence();
                }
            }
            ++g;
        };

#pragma unroll
        for (int i = 0; i < 8; ++i) wa[i] = read_w(g & 1, i);
        xf[0] = read_x(g & 1, 0);
        xf[1] = read_x(g & 1, 1);
        xf[2] = read_x(g & 1, 2);
        // blocks 0, 1, .. cnt-1 (cnt even) alternate W sets (even: wa current)
        for (int j = 0; j < cnt; j += 2) {
            kblock(std::false_type{}, j);
            kblock(std::true_type{}, j + 1);
        }
        if constexpr (!PARTIAL) {
            epilogue(m0, n0, k & 1);
        } else {
            // (the launch has one workgroup per unit, so this is the workgroup's only item and
            // the accumulators are not re-zeroed)
            // A split unit stores its partial sums in accumulator layout: accumulator (i, j) of
            // lane L at (wave * 64 + 8 i + j) * 256 + 4 L of the unit's 65536 floats, one whole
            // KiB per wave store (a buffer descriptor over the wave's 64 KiB, four stores at a
            // time: the 256 accumulators are not all moved to VGPRs at once).
            const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(p.ws + ((int64_t)unit * 4 + wave) * 16384), 0, 65536, kRsrcWord3);
            uint32_t zero;
            asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
            const uint32_t l16 = (__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) + zero) * 16;
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j4 = 0; j4 < 2; ++j4) {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int j = 4 * j4 + jj;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, acc[i][j]), wsr, l16,
                                                               (8 * i + j) * 1024, 0);
                    }
                    settle_stores();
                }
        }
    }
    // No copy may still be writing LDS when the workgroup ends.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
}

// The tile's vectors at (m0, n0) staged in LDS as the main kernel's copies lay them out
// (w_scale, x_scale, bias, then the broadcast gate row or gate_index), by one wave:
// branch-free buffer loads, all in flight at once; entries past N or M read as zeros.
template <int EPI, bool FAST>
__device__ __forceinline__ void stage_tile_vectors(const GemmArgs& p, uint8_t* scal, int64_t m0, int64_t n0, int lane)
{
    const int64_t nn = min(p.N - n0, (int64_t)256), mm = min(p.M - m0, (int64_t)256);
    const __amdgpu_buffer_rsrc_t swr = __builtin_amdgcn_make_buffer_rsrc((void*)(p.sw + n0), 0, (int)(nn * 4), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sxr = __builtin_amdgcn_make_buffer_rsrc((void*)(p.sx + m0), 0, (int)(mm * 4), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.bias ? p.bias + n0 : nullptr), 0, p.bias ? (int)(nn * 2) : 0, kRsrcWord3);
    const bool grow = EPI == VDN_FP8_EPI_GATE && FAST;
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        grow ? (void*)(p.gate + n0) : (void*)(p.gate_index ? p.gate_index + m0 : nullptr), 0,
        grow ? (int)(nn * 2) : (p.gate_index ? (int)(mm * 4) : 0), kRsrcWord3);
    const uint32_t l16 = (uint32_t)lane * 16, l8 = (uint32_t)lane * 8;
    const i32x4_t vsw = __builtin_amdgcn_raw_buffer_load_b128(swr, l16, 0, 0);
    const i32x4_t vsx = __builtin_amdgcn_raw_buffer_load_b128(sxr, l16, 0, 0);
    const i32x2_t vb = __builtin_amdgcn_raw_buffer_load_b64(br, l8, 0, 0);
    const i32x4_t vg4 = grow ? i32x4_t{} : __builtin_amdgcn_raw_buffer_load_b128(gr, l16, 0, 0);
    const i32x2_t vg2 = grow ? __builtin_amdgcn_raw_buffer_load_b64(gr, l8, 0, 0) : i32x2_t{};
    *reinterpret_cast<i32x4_t*>(scal + l16) = vsw;
    *reinterpret_cast<i32x4_t*>(scal + 1024 + l16) = vsx;
    *reinterpret_cast<i32x2_t*>(scal + 2048 + l8) = vb;
    if (grow) *reinterpret_cast<i32x2_t*>(scal + 3072 + l8) = vg2;
    else *reinterpret_cast<i32x4_t*>(scal + 3072 + l16) = vg4;
}

// Last round of a shape that runs whole tiles (no split along K), with at most a quarter of
// the compute units busy in it: each of those 256 x 256 tiles as four 128 x 128 quadrants, one
// workgroup of four waves per quadrant, wave w computing the quadrant's 64 x 64 part
// (columns 64 (w & 1) .., rows 64 (w >> 1) ..) by the main kernel's MFMAs on the same
// fragments, K blocks in the tile's rotated order -- every output the same accumulation,
// so the same bits as the main kernel -- then the same epilogue on its two slabs: four
// times the matrix cores on those tiles (H3 fused QKV [13107, 21504, 5376]: 4368 tiles =
// 17 rounds + 16; small shapes of at most 64 tiles wholly).
// K blocks double-buffered in LDS (X rows, then W rows, the main kernel's row swizzle),
// the next block's copies issued after the barrier that frees its stage. A quadrant moves
// 32 KiB per K block for a quarter of a tile's MFMAs, so the CU's fill rate bounds it:
// about half a tile's time, not a quarter ([1000, 1000, 8192], 16 tiles: 0.039 against
// 0.067 ms; four stages with the next block's fragments read under the MFMAs: 0.049 ms).
// Used only when the quadrants fit one round (at most a quarter of the compute units
// busy in the last round: [2000, 3000, 4096], 96 tiles as 384 quadrant workgroups, took
// 0.045 against 0.042 ms).
template <int EPI, bool FAST>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemm_fp8_quad(GemmArgs p)
{
    using namespace mainloop;
    constexpr int QB = 128;                        // quadrant rows (X) and columns (W)
    constexpr int kQStage = 2 * QB * BK;           // 32 KiB: X rows, then W rows
    __shared__ __attribute__((aligned(1024))) uint8_t qs[2 * kQStage];
    __shared__ __attribute__((aligned(1024))) uint8_t scal[4096];
    __shared__ __attribute__((aligned(16))) uint8_t stg[4 * kStgWave];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int quad = blockIdx.x & 3, r = blockIdx.x >> 2;
    int tm, tn;
    tile_coords(p.t_main + r, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t mq = m0 + QB * (quad >> 1), nq = n0 + QB * (quad & 1);
    if (mq >= p.M || nq >= p.N) return;            // a quadrant wholly past the output
    const int nk = (int)(p.K / BK);
    const int phase = p.k_phase_mod > 0 ? (((tm + tn) % p.k_phase_mod) * p.k_phase_step) % nk : 0;
    if (w == 3) stage_tile_vectors<EPI, FAST>(p, scal, m0, n0, lane);
    // Copies: wave w fills LDS rows 32 w .. 32 w + 31 of the X rows (i < 4) and of the W
    // rows, 8 rows (1 KiB) per copy; lane L lands at row + L/8, physical chunk L%8, so it
    // fetches logical chunk (L%8) ^ row_swizzle(row).
    const i32x4_t xr = rsrc_words(p.xq + mq * p.ldx, min(p.M - mq, (int64_t)QB) * p.ldx);
    const i32x4_t wr = rsrc_words(p.wq + nq * p.ldw, min(p.N - nq, (int64_t)QB) * p.ldw);
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 32 * w + 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ row_swizzle(row);
        xoff[i] = (uint32_t)(row * p.ldx) + c * 16;
        woff[i] = (uint32_t)(row * p.ldw) + c * 16;
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void_t*)qs;
    asm volatile("s_nop 4");   // SGPR write by VALU -> use as a buffer descriptor
    auto copies = [&](int st, int kb) {
        const uint32_t dst = lds_base + (uint32_t)st * kQStage, soff = (uint32_t)kb * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) copy16_to_lds(xr, dst + (32 * w + 8 * i) * BK, xoff[i], soff);
#pragma unroll
        for (int i = 0; i < 4; ++i) copy16_to_lds(wr, dst + (QB + 32 * w + 8 * i) * BK, woff[i], soff);
    };
    // fragments as the main kernel reads them: 16 rows x 128 K bytes, lane L row L % 16,
    // bytes 32 (L / 16) .. + 31 as two 16-byte chunks
    const int fr = lane & 15, fg = lane >> 4;
    auto read_frag = [&](const uint8_t* s, int row) -> i32x8_t {
        const uint4 lo = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg));
        const uint4 hi = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg + 1));
        return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    };
    const int th = w & 1, up = w >> 1;
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{};
    copies(0, phase);
    for (int j = 0; j < nk; ++j) {
        // this wave's copies of block j have landed and its reads of block j - 1 are done;
        // then every wave's, and block j - 1's stage is free for block j + 1
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        __syncthreads();
        if (j + 1 < nk) {
            const int kb = phase + j + 1;
            copies((j + 1) & 1, kb >= nk ? kb - nk : kb);
        }
        const uint8_t* s = qs + (j & 1) * kQStage;
        i32x8_t wf[4], xf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) wf[i] = read_frag(s + QB * BK, 64 * th + 16 * i + fr);
#pragma unroll
        for (int i = 0; i < 4; ++i) xf[i] = read_frag(s, 64 * up + 16 * i + fr);
#pragma unroll
        for (int jx = 0; jx < 4; ++jx)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][jx] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf[jx], acc[i][jx], 0, 0, 0, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __syncthreads();   // the vectors are staged
    // the epilogue of the slabs (th, u = 2 up, 2 up + 1): accumulator (i, j) of this wave
    // is the main kernel's (4 th + i, 4 up + j)
    f32x4_t acc8[8][8];
    auto run = [&](auto tc, auto uc) {
        constexpr int TH = decltype(tc)::value, UP = decltype(uc)::value;
        constexpr int kMask = (3 << (4 * (1 - TH) + 2 - 2 * UP));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc8[4 * TH + i][4 * UP + jj] = acc[i][jj];
        tile_epilogue<EPI, FAST, kMask>(p, scal, stg + w * kStgWave, acc8, m0, n0, quad);
    };
    switch (w) {
        case 0: run(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}); break;
        case 1: run(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}); break;
        case 2: run(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}); break;
        default: run(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}); break;
    }
}

// Split-K reduction: one workgroup of four waves per quadrant of a split tile (four per
// tile). Wave w sums accumulators 16 w .. 16 w + 15 of the quadrant (per lane) over the
// tile's units in slice order (slice 0 + slice 1 + ..., binary32: the order depends only
// on K and the split), two slices' loads in flight at once beside the sums, into LDS; wave
// 3 stages the tile's vectors as the main kernel's copies lay them out; then each wave
// runs the same epilogue for the quadrant's rows 32 w .. 32 w + 31 (its two slabs). Against
// one wave per quadrant holding all 64 accumulators: [3328, 5120, 8192] 0.124 -> 0.113 ms,
// [1000, 1000, 16384] 0.059 -> 0.042 ms, bitwise equal.
template <int EPI, bool FAST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemm_splitk_reduce(GemmArgs p)
{
    using namespace mainloop;
    __shared__ __attribute__((aligned(1024))) uint8_t scal[4096];
    __shared__ __attribute__((aligned(16))) uint8_t stg[4 * kStgWave];
    __shared__ f32x4_t sums[64 * 64];   // [accumulator][lane]
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int quad = blockIdx.x & 3, r = blockIdx.x >> 2;
    int tm, tn;
    tile_coords(p.t_main + r, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    if (w == 3) stage_tile_vectors<EPI, FAST>(p, scal, m0, n0, lane);
    const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.ws + (int64_t)r * p.splits * kUnitFloatsDev + (int64_t)quad * 16384), 0,
        (int)min((int64_t)p.splits * kUnitFloatsDev * 4, (int64_t)0x7fffffff), kRsrcWord3);
    const uint32_t l16 = (uint32_t)lane * 16;
    const int i0 = 16 * w;   // this wave's accumulators i0 .. i0 + 15
    f32x4_t a[16];
#pragma unroll
    for (int q = 0; q < 16; ++q)
        a[q] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wsr, l16, (i0 + q) * 1024, 0));
    for (int sl = 1; sl < p.splits; sl += 2) {
        const bool two = sl + 1 < p.splits;
        // (a missing second slice is read past the descriptor's range: zeros, no traffic)
        const int so = sl * (int)kUnitFloatsDev * 4, so2 = so + (int)kUnitFloatsDev * 4;
        f32x4_t b[16], c[16];
#pragma unroll
        for (int q = 0; q < 16; ++q)
            b[q] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wsr, l16, so + (i0 + q) * 1024, 0));
#pragma unroll
        for (int q = 0; q < 16; ++q)
            c[q] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wsr, l16, so2 + (i0 + q) * 1024, 0));
#pragma unroll
        for (int q = 0; q < 16; ++q) a[q] += b[q];
        if (two) {
#pragma unroll
            for (int q = 0; q < 16; ++q) a[q] += c[q];
        }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) sums[(i0 + q) * 64 + lane] = a[q];
    __syncthreads();
    // wave w: the epilogue's slabs of rows 32 w .. 32 w + 31 (accumulators [.][2 w], [.][2 w + 1])
    f32x4_t acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = sums[(8 * i + j) * 64 + lane];
    uint8_t* const ws = stg + w * kStgWave;
    switch (w) {
        case 0: tile_epilogue<EPI, FAST, 0x88>(p, scal, ws, acc, m0, n0, quad); break;
        case 1: tile_epilogue<EPI, FAST, 0x44>(p, scal, ws, acc, m0, n0, quad); break;
        case 2: tile_epilogue<EPI, FAST, 0x22>(p, scal, ws, acc, m0, n0, quad); break;
        default: tile_epilogue<EPI, FAST, 0x11>(p, scal, ws, acc, m0, n0, quad); break;
    }
}

// ---------------------------------------------------------------------------
// tail kernel: K % 128 != 0 (K % 16 == 0)
// ---------------------------------------------------------------------------
namespace tailloop {
constexpr int BK = 128;
constexpr int kStage = (BM + BN) * BK;
constexpr int kChunks = BM * BK / 16 / kThreads;  // 8
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * BK + ((chunk ^ row_swizzle(row)) << 4); }
}  // namespace tailloop

template <int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemm_fp8_ktail(GemmArgs p)
{
    using namespace tailloop;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStage];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int nk = (int)((p.K + BK - 1) / BK);

    // Thread copies chunk q = tid + 256 i: row q / 8, 16-byte chunk q % 8, through
    // VGPRs (zero past K), into the swizzled LDS layout.
    const __amdgpu_buffer_rsrc_t xr = tile_rsrc(p.xq + m0 * p.ldx, p.M - m0, p.ldx);
    const __amdgpu_buffer_rsrc_t wr = tile_rsrc(p.wq + n0 * p.ldw, p.N - n0, p.ldw);
    const int srow = tid >> 3, schunk = tid & 7;
    auto fill = [&](uint8_t* st, int kt) {
        const uint32_t kb = (uint32_t)kt * BK;
        const bool in = (int64_t)kb + schunk * 16 < p.K;
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int r = srow + 32 * i;
            uint4 vx = z, vw = z;
            if (in) {
                vx = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)(r * p.ldx) + schunk * 16, kb, 0));
                vw = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)(r * p.ldw) + schunk * 16, kb, 0));
            }
            *reinterpret_cast<uint4*>(st + lds_off(r, schunk)) = vx;
            *reinterpret_cast<uint4*>(st + BM * BK + lds_off(r, schunk)) = vw;
        }
    };

    f32x4_t acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int frow = lane & 15, fg = lane >> 4;
    auto read_frag = [&](const uint8_t* s, int row) -> i32x8_t {
        const uint4 lo = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg));
        const uint4 hi = *reinterpret_cast<const uint4*>(s + lds_off(row, 2 * fg + 1));
        return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    };
    for (int kt = 0; kt < nk; ++kt) {
        uint8_t* const st = smem + (kt & 1) * kStage;
        fill(st, kt);
        __syncthreads();
        i32x8_t wf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wf[i] = read_frag(st + BM * BK, wn * 128 + i * 16 + frow);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const i32x8_t xf = read_frag(st, wm * 128 + j * 16 + frow);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf, acc[i][j], 0, 0, 0, 0, 0, 0);
        }
    }

    // Epilogue: lane holds n = n0 + wn*128 + 16 i + 4 (lane/16) + e, m = m0 + wm*128 + 16 j + lane%16.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t m = m0 + wm * 128 + j * 16 + frow;
        if (m >= p.M) continue;
        const float sxm = p.sx[m];
        const uint16_t* grow = gate_row<EPI>(p, m);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t n = n0 + wn * 128 + i * 16 + 4 * fg;
            if (n >= p.N) continue;
            const float a4[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            store4<EPI>(p, m, n, a4, sxm, grow);
        }
    }
}

// K-block rotation of the main kernel: tiles with (tm + tn) odd start one block
// later, so the workgroups sharing an X or W panel do not all miss the same
// lines at once (and strided rows do not hit the same memory channels in
// lockstep). Measured on the QKV and FFN-down shapes; (4, 2) is as good.
constexpr int kPhaseMod = 2, kPhaseStep = 1;

// Tile order for a shape (random codes, one MI355X): m-tile groups of 4 with the K
// rotation for every shape. Groups of 1, 2, 4, 8 on the 16 x 16 x 128 kernel (same
// process, medians of three): FFN-down [32760, 5120, 13824] 1.519 / 1.505 / 1.494 /
// 1.499 ms, attention-out [32760, 5120, 5120] 0.594 / 0.585 / 0.576 / 0.578, H3 FF
// down [13107, 5376, 14336] 0.699 / 0.690 / 0.669 / 0.701, H3 QKV [13107, 21504, 5376]
// 1.147 / 1.062 / 1.032 / 1.040, H3 FF projection [13107, 28672, 5376] 1.499 / 1.389 /
// 1.369 / 1.366 (QKV N = 15360: 1.91 ms against 1.92-1.96 for 2, 8, 16 or no rotation,
// on the earlier 32 x 32 x 64 kernel, which preferred groups of 2 for narrow outputs
// over long rows).
// The K rotation is on for every shape, so the summation order of an output
// depends only on K and on the parity of its tile's (tm + tn): a projection run
// on its own and as a row block of a fused weight (QKV's Wq;Wk;Wv, whose
// widths are multiples of 512) give the same bits. Narrow outputs over short
// rows were 1% faster without it (attention-out [32760, 5120, 5120]: 0.670
// against 0.678 ms).
__host__ inline void tile_order(int64_t N, int64_t K, int& phase_mod, int& group_m)
{
    phase_mod = kPhaseMod;
    group_m = kGroupM;
    (void)N;
    (void)K;
}

// Split of the last partial round along K: for rows of at least 8192 bytes (K), when
// the tiles leave a last round of R <= grid / 2 tiles, each of those R tiles runs as S =
// min(grid / R, nk / 8) K slices on otherwise idle workgroups (at least 8 blocks each),
// then the reduction kernel sums the slices. The H3 FF down projection [13107, 5376,
// 14336]: 1092 tiles = 4 rounds + 68 on 256 CUs, the 68 as 3 slices of 37-38 blocks.
// Projections with shorter rows (the QKV and FF projections) never split, so a fused
// weight's outputs keep the bits of its separate projections.
constexpr int64_t kSplitMinK = 8192;
constexpr int kSplitMinBlocks = 8;
constexpr int64_t kUnitFloats = 65536;   // one 256 x 256 tile of binary32 partial sums

struct SplitPlan {
    int t_main, splits, units;
};

__host__ inline SplitPlan plan_split(int64_t T, int grid, int64_t K)
{
    SplitPlan sp{(int)T, 0, 0};
    if (K < kSplitMinK || K % (2 * mainloop::BK) || grid <= 0) return sp;
    const int64_t R = T % grid;
    if (R == 0 || R > grid / 2) return sp;
    const int64_t S = std::min<int64_t>(grid / R, K / mainloop::BK / kSplitMinBlocks);
    if (S < 2) return sp;
    sp.t_main = (int)(T - R);
    sp.splits = (int)S;
    sp.units = (int)(R * S);
    return sp;
}

}  // namespace

int launch_gated_residual(const uint16_t* residual, int64_t ldr, const uint16_t* gate, int64_t ldgate,
                          const int32_t* gate_index, int64_t gate_rows, const uint16_t* branch, int64_t ldb,
                          uint16_t* out, int64_t ldo, int64_t M, int64_t N, hipStream_t stream);

// Bytes of split-K workspace a [M, N, K] GEMM takes on the current device (0: no split).
int gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t* bytes)
{
    *bytes = 0;
    if (M <= 0 || N <= 0 || K <= 0) return VDN_FP8_OK;
    const int cus = device_cus();
    if (cus <= 0) return set_error(VDN_FP8_ELAUNCH, "gemm: cannot query the device's compute units");
    const int64_t T = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (T > (int64_t)INT32_MAX / 2) return VDN_FP8_OK;
    const SplitPlan sp = plan_split(T, cus, K);
    *bytes = (int64_t)sp.units * kUnitFloats * (int64_t)sizeof(float);
    return VDN_FP8_OK;
}

// The GEMM with an optional split-K workspace (ws NULL: no split).
int gemm_launch(const void* xq, const float* x_scale, const void* wq, const float* w_scale, int64_t M, int64_t N,
                int64_t K, int64_t ldx, int64_t ldw, const void* bias, int epilogue, const void* gate,
                const int32_t* gate_index, int64_t gate_rows, int64_t ldgate, const void* residual, int64_t ldres,
                void* out, int64_t ldo, float* ws, int64_t ws_bytes, hipStream_t stream)
{
    if (M < 0 || N < 0 || K < 0) return set_error(VDN_FP8_EINVAL, "gemm: negative shape");
    if (M == 0 || N == 0) return VDN_FP8_OK;
    if (K == 0 || K % 16) return set_error(VDN_FP8_EINVAL, "gemm: K must be a positive multiple of 16 (K=%lld)", (long long)K);
    if (N % 4) return set_error(VDN_FP8_EINVAL, "gemm: N must be a multiple of 4 (N=%lld)", (long long)N);
    if (!xq || !wq || !x_scale || !w_scale || !out) return set_error(VDN_FP8_EINVAL, "gemm: null pointer");
    if (ldx < K || ldw < K || ldo < N || ldx % 16 || ldw % 16 || ldo % 4)
        return set_error(VDN_FP8_EINVAL, "gemm: need ldx, ldw >= K and multiples of 16, ldo >= N and a multiple of 4");
    if (ldx * 256 > (int64_t)0x7fffffff || ldw * 256 > (int64_t)0x7fffffff)
        return set_error(VDN_FP8_EINVAL, "gemm: row stride too large (256 rows must span < 2 GiB)");
    if (!aligned(xq, 16) || !aligned(wq, 16) || !aligned(out, 8) || !aligned(w_scale, 16) || !aligned(x_scale, 16) ||
        (bias && !aligned(bias, 16)) || (gate_index && !aligned(gate_index, 16)))
        return set_error(VDN_FP8_EINVAL, "gemm: misaligned operand (xq, wq, x_scale, w_scale, bias, gate_index 16 B; out 8 B)");
    if (epilogue == VDN_FP8_EPI_GATE) {
        if (!gate || gate_rows < 1) return set_error(VDN_FP8_EINVAL, "gemm: the gate epilogue needs a gate table of >= 1 row");
        if (ldgate < N || ldgate % 4 || !aligned(gate, 8)) return set_error(VDN_FP8_EINVAL, "gemm: gate rows must be >= N and 8-byte aligned");
        if (residual && (ldres < N || ldres % 4 || !aligned(residual, 8)))
            return set_error(VDN_FP8_EINVAL, "gemm: residual rows must be >= N and 8-byte aligned");
    } else if (epilogue == VDN_FP8_EPI_F32) {
        if (bias || gate || residual || gate_index)
            return set_error(VDN_FP8_EINVAL, "gemm: the binary32 output takes no bias, gate or residual");
        if (!aligned(out, 16)) return set_error(VDN_FP8_EINVAL, "gemm: the binary32 output must be 16-byte aligned");
    } else if (epilogue != VDN_FP8_EPI_NONE && epilogue != VDN_FP8_EPI_GELU_TANH) {
        return set_error(VDN_FP8_EINVAL, "gemm: unknown epilogue %d", epilogue);
    }
    if (ws_bytes < 0 || (ws && !aligned(ws, 16))) return set_error(VDN_FP8_EINVAL, "gemm: workspace must be 16-byte aligned");
    const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if (tiles_m * tiles_n > (int64_t)INT32_MAX / 2) return set_error(VDN_FP8_EINVAL, "gemm: problem too large");
    const int64_t T = tiles_m * tiles_n;
    GemmArgs p{(const uint8_t*)xq, x_scale, (const uint8_t*)wq, w_scale, M, N, K, ldx, ldw,
               (const uint16_t*)bias, (const uint16_t*)gate, gate_index, gate_rows, ldgate,
               (const uint16_t*)residual, ldres, (uint16_t*)out, ldo, (int)tiles_m, (int)tiles_n,
               kPhaseMod, kPhaseStep, kGroupM, (int)T, 0, 0, nullptr};
    tile_order(N, K, p.k_phase_mod, p.group_m);
    const bool main = (K % (2 * mainloop::BK)) == 0;
    int64_t blocks = T;
    if (main) {
        const int cus = device_cus();
        if (cus <= 0) return set_error(VDN_FP8_ELAUNCH, "gemm: cannot query the device's compute units");
        if (ws) {
            const SplitPlan sp = plan_split(T, cus, K);
            const int64_t need = (int64_t)sp.units * kUnitFloats * (int64_t)sizeof(float);
            if (ws_bytes < need)
                return set_error(VDN_FP8_EINVAL, "gemm: workspace of %lld bytes, this shape needs %lld",
                                 (long long)ws_bytes, (long long)need);
            if (sp.units) {
                p.t_main = sp.t_main;
                p.splits = sp.splits;
                p.units = sp.units;
                p.ws = ws;
            }
        }
        if (!p.units) {
            // a last round of at most a quarter of the compute units as quadrants
            const int64_t R = T % cus;
            if (R > 0 && 4 * R <= cus) p.t_main = (int)(T - R);   // tiles t_main .. T - 1: k_gemm_fp8_quad
        }
        blocks = std::min<int64_t>((int64_t)p.t_main, cus);
    }
    const dim3 grid((unsigned)std::max<int64_t>(blocks, 1)), block(kThreads);
    const dim3 ugrid((unsigned)std::max(p.units, 1)), rgrid((unsigned)(p.units ? 4 * (p.units / p.splits) : 1));
    const dim3 rblock(256);
    // (no split: the tiles past t_main run as quadrants)
    const int quads = p.units ? 0 : (int)(T - p.t_main);
    const dim3 qgrid((unsigned)std::max(4 * quads, 1));
    // the fast epilogue: 16-byte output rows, row offsets within 31 bits, and no
    // per-row gate or residual (a gate table of one row is staged like the bias)
    const bool gate_broadcast = epilogue == VDN_FP8_EPI_GATE && !residual && (gate_rows == 1 || !gate_index) &&
                                aligned(gate, 16);
    const bool out16 = N % 8 == 0 && ldo % 8 == 0 && aligned(out, 16) && (int64_t)BM * ldo * 2 <= (int64_t)0x7fffffff;
    const bool fast = (epilogue != VDN_FP8_EPI_GATE || gate_broadcast) && out16;
    // A per-row gate or a residual on 16-byte rows: the fast epilogue with the gate and
    // the residual applied in its row layout, bf16(residual + gate[i] * v), the gated
    // residual kernel's arithmetic (H3 FF down [13107, 5376, 14336] with a gate table
    // and the residual: 0.750 -> 0.691 ms against the GEMM writing v and that kernel
    // reading it back; [32760, 5120, 13824] 1.628 -> 1.532 ms; bitwise equal). Row
    // offsets past 31 bits keep the two kernels.
    const bool row_gate = main && epilogue == VDN_FP8_EPI_GATE && !gate_broadcast && out16 && aligned(gate, 16) &&
                          ldgate % 8 == 0 && (!residual || (aligned(residual, 16) && ldres % 8 == 0));
    if (row_gate && (!residual || (int64_t)BM * ldres * 2 <= (int64_t)0x7fffffff) &&
        gate_rows * ldgate * 2 <= (int64_t)0x7fffffff) {
        if (p.t_main) hipLaunchKernelGGL((k_gemm_fp8<kEpiRowGate, true, false>), grid, block, 0, stream, p);
        if (quads) hipLaunchKernelGGL((k_gemm_fp8_quad<kEpiRowGate, true>), qgrid, block, 0, stream, p);
        if (p.units) {
            hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, true>), ugrid, block, 0, stream, p);
            hipLaunchKernelGGL((k_gemm_splitk_reduce<kEpiRowGate, true>), rgrid, rblock, 0, stream, p);
        }
        return check_launch("gemm");
    }
    if (row_gate) {
        if (p.t_main) hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, false>), grid, block, 0, stream, p);
        if (quads) hipLaunchKernelGGL((k_gemm_fp8_quad<VDN_FP8_EPI_NONE, true>), qgrid, block, 0, stream, p);
        if (p.units) {
            hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, true>), ugrid, block, 0, stream, p);
            hipLaunchKernelGGL((k_gemm_splitk_reduce<VDN_FP8_EPI_NONE, true>), rgrid, rblock, 0, stream, p);
        }
        const int st = check_launch("gemm");
        if (st != VDN_FP8_OK) return st;
        return launch_gated_residual((const uint16_t*)residual, ldres, (const uint16_t*)gate, ldgate, gate_index,
                                     gate_rows, (const uint16_t*)out, ldo, (uint16_t*)out, ldo, M, N, stream);
    }
#define VDN_LAUNCH(E)                                                                                    \
    do {                                                                                                 \
        if (main && fast) {                                                                              \
            if (p.t_main) hipLaunchKernelGGL((k_gemm_fp8<E, true, false>), grid, block, 0, stream, p);   \
            if (quads) hipLaunchKernelGGL((k_gemm_fp8_quad<E, true>), qgrid, block, 0, stream, p);     \
            if (p.units) {                                                                               \
                hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, true>), ugrid, block, 0, stream, p); \
                hipLaunchKernelGGL((k_gemm_splitk_reduce<E, true>), rgrid, rblock, 0, stream, p);        \
            }                                                                                            \
        } else if (main) {                                                                               \
            if (p.t_main) hipLaunchKernelGGL((k_gemm_fp8<E, false, false>), grid, block, 0, stream, p);  \
            if (quads) hipLaunchKernelGGL((k_gemm_fp8_quad<E, false>), qgrid, block, 0, stream, p);    \
            if (p.units) {                                                                               \
                hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, true>), ugrid, block, 0, stream, p); \
                hipLaunchKernelGGL((k_gemm_splitk_reduce<E, false>), rgrid, rblock, 0, stream, p);       \
            }                                                                                            \
        } else {                                                                                         \
            hipLaunchKernelGGL((k_gemm_fp8_ktail<E>), grid, block, 0, stream, p);                        \
        }                                                                                                \
    } while (0)
    if (epilogue == VDN_FP8_EPI_F32) {
        // (the general epilogue only: the fast one stages bf16 rows)
        if (main) {
            if (p.t_main) hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_F32, false, false>), grid, block, 0, stream, p);
            if (quads) hipLaunchKernelGGL((k_gemm_fp8_quad<VDN_FP8_EPI_F32, false>), qgrid, block, 0, stream, p);
            if (p.units) {
                hipLaunchKernelGGL((k_gemm_fp8<VDN_FP8_EPI_NONE, true, true>), ugrid, block, 0, stream, p);
                hipLaunchKernelGGL((k_gemm_splitk_reduce<VDN_FP8_EPI_F32, false>), rgrid, rblock, 0, stream, p);
            }
        } else {
            hipLaunchKernelGGL((k_gemm_fp8_ktail<VDN_FP8_EPI_F32>), grid, block, 0, stream, p);
        }
        return check_launch("gemm");
    }
    switch (epilogue) {
        case VDN_FP8_EPI_NONE: VDN_LAUNCH(VDN_FP8_EPI_NONE); break;
        case VDN_FP8_EPI_GELU_TANH: VDN_LAUNCH(VDN_FP8_EPI_GELU_TANH); break;
        default: VDN_LAUNCH(VDN_FP8_EPI_GATE); break;
    }
#undef VDN_LAUNCH
    return check_launch("gemm");
}
}  // namespace vdn

using namespace vdn;

extern "C" int vdn_fp8_gemm(const void* xq, const float* x_scale, const void* wq, const float* w_scale, int64_t M,
                            int64_t N, int64_t K, int64_t ldx, int64_t ldw, const void* bias, int epilogue,
                            const void* gate, const int32_t* gate_index, int64_t gate_rows, int64_t ldgate,
                            const void* residual, int64_t ldres, void* out, int64_t ldo, hipStream_t stream)
{
    return gemm_launch(xq, x_scale, wq, w_scale, M, N, K, ldx, ldw, bias, epilogue, gate, gate_index, gate_rows,
                       ldgate, residual, ldres, out, ldo, nullptr, 0, stream);
}

extern "C" int vdn_fp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int64_t* bytes)
{
    if (!bytes) return set_error(VDN_FP8_EINVAL, "gemm_workspace_size: null pointer");
    return gemm_workspace_bytes(M, N, K, bytes);
}

extern "C" int vdn_fp8_gemm_ws(const void* xq, const float* x_scale, const void* wq, const float* w_scale, int64_t M,
                               int64_t N, int64_t K, int64_t ldx, int64_t ldw, const void* bias, int epilogue,
                               const void* gate, const int32_t* gate_index, int64_t gate_rows, int64_t ldgate,
                               const void* residual, int64_t ldres, void* out, int64_t ldo, void* workspace,
                               int64_t workspace_bytes, hipStream_t stream)
{
    return gemm_launch(xq, x_scale, wq, w_scale, M, N, K, ldx, ldw, bias, epilogue, gate, gate_index, gate_rows,
                       ldgate, residual, ldres, out, ldo, (float*)workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// The allocation-free GEMM: the split-K workspace in a static device array
// ---------------------------------------------------------------------------
// Largest split workspace on a 256-CU part: units <= compute units, 256 KiB each.
constexpr int64_t kScratchBytes = 64LL << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxScratchDevices];   // this device's copy of `scratch`, or null before the first call

// The device address of `scratch` on the current device, looked up on the first call on
// each device (the host-side name is not a device address); null if the lookup fails.
float* scratch_ptr(int dev)
{
    if (dev < 0 || dev >= kMaxScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch[dev] = static_cast<float*>(ptr);
    }
    return g_scratch[dev];
}
}  // namespace

extern "C" int vdn_fp8_gemm_noalloc(const void* xq, const float* x_scale, const void* wq, const float* w_scale,
                                    int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw, const void* bias,
                                    int epilogue, const void* gate, const int32_t* gate_index, int64_t gate_rows,
                                    int64_t ldgate, const void* residual, int64_t ldres, void* out, int64_t ldo,
                                    hipStream_t stream)
{
    int64_t need = 0;
    const int st = gemm_workspace_bytes(M, N, K, &need);
    if (st != VDN_FP8_OK) return st;
    if (need > kScratchBytes)
        return set_error(VDN_FP8_EINVAL, "gemm_noalloc: this shape's split workspace (%lld bytes) exceeds the "
                                         "static scratch of %lld bytes", (long long)need, (long long)kScratchBytes);
    float* ws = nullptr;
    if (need > 0) {
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess) return set_error(VDN_FP8_ELAUNCH, "gemm_noalloc: no current device");
        ws = scratch_ptr(dev);
        if (!ws) return set_error(VDN_FP8_ELAUNCH, "gemm_noalloc: cannot look up the scratch array on device %d", dev);
    }
    return gemm_launch(xq, x_scale, wq, w_scale, M, N, K, ldx, ldw, bias, epilogue, gate, gate_index, gate_rows,
                       ldgate, residual, ldres, out, ldo, ws, ws ? kScratchBytes : 0, stream);
}
