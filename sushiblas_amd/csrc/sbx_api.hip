// sbx_api.hip -- the C ABI (include/sbx.h): argument validation, the
// column-major -> row-major mapping, quick returns, and the tiling heuristics
// that choose a kernel.  This is what gemm_dispatch<T>
// (src/ops/blas/level3/gemm.cpp:44-79) does in the reference, with oneMKL's
// internal kernel choice replaced by an explicit, inspectable one.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/sbx.h"
#include "gemv.hpp"
#include "launch.hpp"
#ifdef SBX_PROBE
#include "sbx_probe.h"
#endif

namespace sbx {

hipError_t launch_fill_uniform(int dtype, void* out, int64_t n, uint64_t seed, uint32_t stream,
                               hipStream_t s);
hipError_t launch_fill_normal(int dtype, void* out, int64_t n, uint64_t seed, uint32_t stream,
                              double scale, hipStream_t s);

namespace {

constexpr int64_t kMaxDim = (int64_t)1 << 30;        // m, n, k limit (int32 tile math)
constexpr int64_t kMaxGridZ = 65535;                  // batch chunk per launch

struct Problem {
    int dtype;
    bool ta, tb;
    int64_t m, n, k;
    const void* A;
    int64_t lda, str_a;
    const void* B;
    int64_t ldb, str_b;
    void* C;
    int64_t ldc, str_c;
    int64_t batch;
    int relu;  // fused ReLU epilogue
    int uplo;  // 0: whole C; 1 / 2: lower / upper triangle only (SYRK, B == A, m == n)
    // grouped launch: batch entry z's A, B, C come from this device table
    // (3 pointers per entry); A/B/C above are then 16-byte aligned (or not)
    // stand-in addresses that only carry the alignment fact C's vector
    // stores need
    const void* const* table;
    int table_swap;
};

// Tile configurations compiled into the library (gemm_cfg_*.hip).
enum Cfg {
    F32_256x256,   // large fp32: 8 waves of 64x128, 2 waves/SIMD (128 accumulators)
    F32_256x128,   // large fp32: 4 waves of 64x128, two workgroups per CU, 2 tiles in flight
    F32_128x128,   // mid-size fp32: 4 waves of 64x64, 2 waves/SIMD, 2 tiles in flight
    F32_128x128_O3,  // the same tile at 3 waves/SIMD (three workgroups per CU)
    F32_128x64,    // n <= 64 (tall-skinny): 4 waves of 64x32, 2 tiles in flight
    F32_256x64,    // n <= 64 with a full round of 256-row tiles: 8 waves of 32x64 (16x16x4 MFMAs)
    F32_256x48,    // 32 < n <= 48: the 256x64 tile computing 48 columns (waves of 32x48)
    F32_64x128,    // m <= 64
    F32_64x256,    // m <= 64 with a full round of 256-column tiles: 8 waves of 64x32 (16x16x4 MFMAs)
    F32_48x256,    // 32 < m <= 48: the 64x256 tile computing 48 rows (waves of 48x32)
    F32_128x32,    // n <= 32: 4 waves of 32x32 (16x16x4 MFMAs)
    F32_32x128,    // m <= 32: 4 waves of 32x32 (16x16x4 MFMAs)
    F32_64x64,     // fp32 mid-size: 4 waves of 32x32
    F64_128x128,   // fp64: 4 waves of 64x64, 2 waves/SIMD
    F64_128x64,
    F64_64x128,
    F64_64x64,     // fp64 mid-size: 4 waves of 32x32
    F32_SMALL,     // small problems: 32x32 tiles, K cut over the 4 waves (gemm_small.hip)
    F64_SMALL,
    F32_SMALL8,    // the same with K cut over 8 waves
    GENERIC,
};

struct CfgInfo {
    const char* name;
    int bm, bn, bk;
    int per_cu;  // resident workgroups per CU
};

const CfgInfo kCfg[] = {
    {"mfma_f32_256x256x32_w4x2", 256, 256, 32, 1}, {"mfma_f32_256x128x16_w4x1", 256, 128, 16, 2},
    {"mfma_f32_128x128x16_w2x2", 128, 128, 16, 2},
    {"mfma_f32_128x128x16_w2x2_o3", 128, 128, 16, 3},
    {"mfma_f32_128x64x32_w2x2", 128, 64, 32, 2},   {"mfma_f32_256x64x32_w8x1", 256, 64, 32, 1},
    {"mfma_f32_256x48x32_w8x1", 256, 64, 32, 1},  // bn: the loaded (and workspace) width
    {"mfma_f32_64x128x32_w2x2", 64, 128, 32, 2},   {"mfma_f32_64x256x32_w1x8", 64, 256, 32, 1},
    {"mfma_f32_48x256x32_w1x8", 64, 256, 32, 1},  // bm: the loaded (and workspace) height
    {"mfma_f32_128x32x32_w4x1", 128, 32, 32, 2},   {"mfma_f32_32x128x32_w1x4", 32, 128, 32, 2},
    {"mfma_f32_64x64x32_w2x2", 64, 64, 32, 2},
    {"mfma_f64_128x128x16_w2x2", 128, 128, 16, 2}, {"mfma_f64_128x64x16_w2x2", 128, 64, 16, 2},
    {"mfma_f64_64x128x16_w2x2", 64, 128, 16, 2},   {"mfma_f64_64x64x16_w2x2", 64, 64, 16, 2},
    {"mfma_f32_32x32_ksplit4", 32, 32, 32, 1},
    {"mfma_f64_32x32_ksplit4", 32, 32, 32, 1},     {"mfma_f32_32x32_ksplit8", 32, 32, 32, 1},
    {"generic_64x64x16", 64, 64, 16, 4},
};
static_assert(sizeof(kCfg) / sizeof(kCfg[0]) == GENERIC + 1, "one kCfg entry per Cfg, in order");

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The small-problem kernel's forms (gemm_small.hip).
inline bool is_small(Cfg c)
{
    return c == F32_SMALL || c == F64_SMALL || c == F32_SMALL8;
}

// Tile configurations worth modelling for a problem, the default first; cus
// is the device's CU count (the round size of one-per-CU tiles).  *large is
// set for the large-fp32 candidates, whose model adds an epilogue term.  At
// most kMaxCands are written (the fp32 branch of mid-size shapes has seven).
constexpr int kMaxCands = 7;
int candidate_cfgs(int dtype, int64_t m, int64_t n, int uplo, int64_t cus, Cfg* out, bool* large)
{
    *large = false;
    if (uplo) {
        // a triangle needs square tiles, so diagonal tiles are the tm == tn ones
        if (dtype != SBX_F32) {
            out[0] = F64_128x128;
            return 1;
        }
        int c = 0;
        const int64_t t = cdiv(n, 256);
        if (t * (t + 1) / 2 >= cus) out[c++] = F32_256x256;
        // the order breaks exact ties of the model only
        out[c++] = F32_128x128_O3;
        out[c++] = F32_128x128;
        return c;
    }
    const bool f32 = dtype == SBX_F32;
    const Cfg sq = f32 ? F32_128x128 : F64_128x128;
    const Cfg tall = f32 ? F32_128x64 : F64_128x64;   // n <= 64 (tall-skinny)
    const Cfg wide = f32 ? F32_64x128 : F64_64x128;   // m <= 64
    int c = 0;
    if (n <= 64) {
        // n <= 32: a 64-wide tile would spend half its MFMAs on padding,
        // where a 32-wide one streams A at up to 5.9 TB/s (65536 x 32 x
        // 4096: 183 against 272 us; 40000 x 32 x 2048: 76 against 85 us)
        if (f32 && n <= 32) out[c++] = F32_128x32;
        // 32 < n <= 48: the 256-row tile computing 48 of its 64 columns, 3/4
        // of the MFMAs of the 64-wide tiles (65536 x 48 x 4096: 263 us on
        // 256x64 against 218 for the vendor)
        if (f32 && n > 32 && n <= 48) out[c++] = F32_256x48;
        // one 8-wave 256-row workgroup per CU: B is read by half as many
        // workgroups (65536 x 64 x 4096: 291-294 us against 296-300)
        if (f32 && cdiv(m, 256) >= cus) out[c++] = F32_256x64;
        out[c++] = tall;
        // last, so that ties keep the tiles above: m <= 64 too (a batch of
        // 64^3 problems: 128x64 spends half its MFMAs on padding).  fp64
        // only where m <= 64 as well: 512 x 64^3 11.4 against 14.8 us,
        // 64 x 64 x 8192 +splitk31 16.0 against 23.9 us; with a long m the
        // small-problem kernel or 128x64 stays ahead (40000 x 32 x 2048:
        // 152 against 179 us, 24 x 100000 x 1024: 183 against 211 us)
        if (f32 || m <= 64) out[c++] = f32 ? F32_64x64 : F64_64x64;
    } else if (m <= 64) {
        // the mirror of the tall case (column-major tall-skinny calls land
        // here): 64 x 65536 x 4096 270-272 against 280-284 us for 64x128
        if (f32 && m <= 32) out[c++] = F32_32x128;  // (32 x 65536 x 4096: 166 against 245 us)
        // the mirror of the 48-column tile
        if (f32 && m > 32 && m <= 48) out[c++] = F32_48x256;
        if (f32 && cdiv(n, 256) >= cus) out[c++] = F32_64x256;
        out[c++] = wide;
        if (f32) out[c++] = F32_64x64;
    } else if (f32 && cdiv(m, 256) * cdiv(n, 256) >= cus * 3 / 4) {
        // Large fp32.  Two 256x128 workgroups per CU (64x128 per wave)
        // overlap each other's prologue and epilogue; they beat the 256^2
        // tile, which runs alone on its CU, on all 15 shapes timed (8192^3
        // 7211 vs 7277 us, 12288 x 8192 x 1024 1405 vs 1468 us), so the
        // 256^2 tile is left to SYRK.  They lead where their grid is (nearly)
        // whole rounds; elsewhere the 128^2 tile at two per CU, whose finer
        // grid and split tail land closer to whole rounds, comes first
        // (5000^2 x 1000: 376 against 422 us, 5120^3: 1786 against 1872 us).
        *large = true;
        const int64_t slots = 2 * cus, left = cdiv(m, 256) * cdiv(n, 128) % slots;
        const bool whole = left == 0 || left >= slots * 7 / 8;
        if (whole) out[c++] = F32_256x128;
        out[c++] = F32_128x128;
        if (!whole) out[c++] = F32_256x128;
        // three 128^2 workgroups per CU: one whole round of 4095 x 3001 x
        // 2047's 768 tiles
        out[c++] = F32_128x128_O3;
    } else {
        out[c++] = sq;
        if (f32) out[c++] = F32_128x128_O3;
        // fp64 mid-size: four 64^2 tiles per 128^2 (1024^3 NN 36 against
        // 52 us on the small-problem kernel; 1536^3 +splitk4 107 against
        // 137 us for 128^2 +splitk3)
        if (!f32) out[c++] = F64_64x64;
        // the two 64-wide tiles model alike; measured, 64x128 is the faster
        // one on most square-ish shapes, so it comes first
        out[c++] = wide;
        out[c++] = tall;
        // fp32 mid-size: 64^2 tiles, after 64x128, which wins the shapes the
        // model rates alike (2048^3: 121 against 127 us); 1024^3 NN 20
        // against 27 us on the small-problem kernel, 1536^3 +splitk4 60
        // against 73 us for 128^2 +splitk3
        if (f32) out[c++] = F32_64x64;
    }
    out[c++] = f32 ? F32_SMALL : F64_SMALL;
    // the 8-wave form cuts K over twice the waves: it shortens each wave's
    // chain of dependent loads where few tiles share a CU (512^3: 6.45 ->
    // 6.19 us, 256^2 x 4096: 37.6 -> 29.2 us)
    if (f32) out[c++] = F32_SMALL8;
    return c;
}

// Largest byte offset an MFMA tile forms relative to its buffer base.
bool offsets_fit(bool kc, int tile_x, int bk, int64_t ld, size_t elem)
{
    const int64_t rows = kc ? tile_x : bk;
    const int64_t span = (rows * ld + (kc ? bk : tile_x)) * (int64_t)elem;
    return span < (int64_t)0x7ffffff0 - 64;
}

bool mfma_feasible(const Problem& p, Cfg c)
{
    const CfgInfo& ci = kCfg[c];
    // the small-problem kernel's grid is (tiles along m, tiles along n, batch)
    if (is_small(c) && cdiv(p.n, ci.bn) > 65535)
        return false;
    // computes 48 columns of its single tile column
    if (c == F32_256x48 && p.n > 48) return false;
    if (c == F32_48x256 && p.m > 48) return false;  // and of rows
    const size_t elem = p.dtype == SBX_F32 ? 4 : 8;
    return offsets_fit(!p.ta, ci.bm, ci.bk, p.lda, elem) &&
           offsets_fit(p.tb, ci.bn, ci.bk, p.ldb, elem) &&
           cdiv(p.m, ci.bm) * cdiv(p.n, ci.bn) < ((int64_t)1 << 31);
}

int check_ld(int layout, bool trans, int64_t rows, int64_t cols, int64_t ld)
{
    // stored matrix is rows x cols of op(X)^T if trans
    const int64_t sr = trans ? cols : rows, sc = trans ? rows : cols;
    const int64_t need = layout == 0 ? sc : sr;
    return ld >= (need > 1 ? need : 1) ? SBX_OK : SBX_INVALID_ARGUMENT;
}

// ---------------------------------------------------------------------------
// Kernel choice and split-K: the candidate plan (tile config x split) with
// the least modelled time.  The tile configs' constants were fitted (bounded
// least squares on log time, robust loss) to every candidate plan of 323
// problems timed on MI355X, 14008 plan timings: bench.py's
// regret_shapes(seed, 70) for seeds 101, 102 and 103 (fp32 and fp64, both
// layouts and all four transposes, a quarter of them batched, 1e8 .. 4e11
// flops), 24 SYRK problems of regret_syrk_shapes(101, 24), and 89 fixed
// problems (the benchmark's shapes, the selection tests' shapes: large,
// tall, wide and long-K ones, batches of small ones, SYRK).  The
// small-problem kernel's terms were refitted later on their own (see
// small_seconds).
//   * a tile config keeps P workgroups per CU (its waves per SIMD); a
//     workgroup's time is w = 2*BM*BN*K_part / (R * eff) + kTileSec +
//     (C tile bytes) / kTileStoreBw, R per dtype, eff per config;
//   * a round of P*CUs workgroups takes P*w; a partial round whose busiest
//     CU holds q < P workgroups takes q*w/e1, e1 what a CU achieves short of
//     its co-resident partners;
//   * the grid adds F once (pipeline fill and the last epilogue; in between,
//     co-resident workgroups hide each other's);
//   * a split adds the reduction kernel and the partial round trip, G +
//     (partial bytes the reduction reads) / W, and each part kPartSec;
//   * the one-launch small-problem kernel is modelled on its own (see
//     small_seconds).
// Whole rounds run unsplit; only the tail (T mod P*CUs tiles, or all of them)
// may be cut into s k-ranges of at least two k tiles each, s from kSplitSet;
// a split is taken if predicted >= 0.5 % faster than the fewer ranges before it.
// Split partials live in a workspace cached per (device, stream): calls on
// one stream are ordered, so they can share it; the first call that needs
// more memory grows it (the only allocation on the GEMM path; outgrown
// buffers are kept, see WorkspaceLease).  The reduction sums the parts in
// fixed order, so results are deterministic.
// ---------------------------------------------------------------------------
constexpr int kMaxSplit = kMaxSplitParts;

struct SplitPlan {
    int num_full;
    int split;
    int rem;
};

struct Choice {
    Cfg cfg;
    SplitPlan sp;
    double seconds;  // model prediction
};

int64_t tile_count(const Problem& p, Cfg c)
{
    const CfgInfo& ci = kCfg[c];
    if (p.uplo) {
        const int64_t t = cdiv(p.n, ci.bn);
        return t * (t + 1) / 2;
    }
    return cdiv(p.m, ci.bm) * cdiv(p.n, ci.bn);
}

// Modelled time of `units` workgroups of `work` seconds each.
double rounds_time(int64_t units, double work, int64_t per_cu, int64_t cus, double e1)
{
    if (units <= 0) return 0.0;
    const int64_t slots = per_cu * cus;
    double t = (double)(units / slots) * (double)per_cu * work;
    const int64_t left = units % slots;
    if (left) {
        const int64_t q = cdiv(left, cus);
        t += (double)q * work / (q == per_cu ? 1.0 : e1);
    }
    return t;
}

// Fitted constants of the tile configs (per CU, seconds, bytes per second).
constexpr double kRateF32 = 5.926e11;
constexpr double kRateF64 = 2.964e11;
constexpr double kGridSec = 4.409e-6;     // F
constexpr double kReduceSec = 3.112e-6;   // G
constexpr double kReduceBw = 3.711e12;    // W
constexpr double kPartSec = 8.200e-7;
constexpr double kTileSec = 7.824e-7;
constexpr double kTileStoreBw = 2.2870e10;
constexpr double kE1 = 0.9944;
// The same for the 32-wide tiles, which stream their long operand from HBM:
// alone on a CU a workgroup cannot pull the CU's share of the bandwidth
// (8192 x 16 x 8192: split in four, one workgroup per CU, 57 us; in eight,
// two per CU, 51 us, though the split costs more to reduce).
constexpr double kE1Stream = 0.8;

// Relative MFMA rate of a tile config.  1 for the 128^2 tiles, which the
// rates are quoted on, for the configs only tall, wide or large shapes reach,
// and for the fp64 128x64 and 64x128 tiles, whose fitted factors (1.005,
// 1.001) left the cross-validated regret unchanged when fixed at 1 (and
// moved the fp64 8192^3 pick off the 128^2 tile, 14630 against 14400 us).
double cfg_eff(Cfg c)
{
    switch (c) {
    case F32_128x128_O3: return 1.0091;
    case F32_128x64: return 0.9656;
    // the model counts the loaded 64 columns, of which 48 are computed: at
    // 65536 x {33, 40, 48} x 4096 it ran 0.85-0.86 of the 256x64 tile's time
    case F32_256x48: return 1.17;
    case F32_48x256: return 1.17;  // its mirror, the same counting
    case F32_64x128: return 0.9732;
    case F32_64x64: return 0.9478;
    case F32_256x128: return 1.0157;
    case F64_64x64: return 0.9837;
    default: return 1.0;
    }
}

// Large fp32 shapes (epi set): the part of a tile's epilogue the CU's other
// workgroups do not hide, kEpiSec per byte of the C tile, times 12 for C rows
// that take no vector access (single-element loads and stores), and per
// split part kEpiSec per byte of its partial; both times 0.2 at three
// workgroups per CU.
constexpr double kEpiSec = 2.2496e-13;

// The small-problem kernel (one launch of 32x32 tiles, w = 2*32*32*K flops
// each), per form -- fp32 with K cut over 4 or 8 waves, fp64 over 4: a
// launch cost `sec`; a workgroup alone on a CU computes at `rs`, up to `occ`
// of them overlap on one CU, and past that the CU's rate `rc` limits; each
// workgroup adds `wg`; the operand bytes over kSmallBw (kSmallBwBatch for a
// batch, whose entries' slabs are contiguous) bound the time from below.
// Its waves read operands straight from memory in the MFMA lane layout, so
// the cost per k depends on which operands are k-contiguous: the layout
// factors scale the flops per [A k-contiguous][B k-contiguous].
// Fitted (robust least squares on log time, the tile constants above held)
// to 28,488 plan timings of 617 problems, timed on the kernel as it is:
// regret_shapes(seed, 70) for seeds 101-103, regret_shapes(seed, 60) for
// seeds 20261203, 20261207, 20261209 and 20261211, the 57 problems of the
// selection tests and 110 problems with one side of 48-512 and the other of
// 512-8192.  A plan's residual weighs more when the plan is near its
// problem's fastest in measured time or in the fitted model's prediction
// (refitted three times): a plan the model rates too fast misleads the
// choice as much as the fastest rated too slow.
struct SmallForm {
    double sec, wg, rs, rc;
    int occ;
};
constexpr SmallForm kSmallF32W4{2.8336e-06, 4.5870e-07, 2.9187e+11, 3.4076e+11, 2};
constexpr SmallForm kSmallF32W8{2.7012e-06, 5.0971e-07, 4.8464e+11, 3.5333e+11, 1};
constexpr SmallForm kSmallF64W4{3.1395e-06, 1.0982e-06, 4.2042e+11, 1.8879e+11, 2};
constexpr double kSmallLayF32[2][2] = {{1.0, 1.0856}, {0.9772, 1.0096}};
constexpr double kSmallLayF64[2][2] = {{1.0, 1.0486}, {1.0604, 0.9434}};
constexpr double kSmallBw = 4.5975e+12;
constexpr double kSmallBwBatch = 7.1474e+12;

// The split-K space of a tile config: whole rounds run unsplit, and the
// `rem` tiles of the tail (every tile of every entry, for a batch whose grid
// fills less than one round) may be cut into 2 .. smax k-ranges of at least
// two k tiles each.  smax == 0: no split (the small-problem and generic
// kernels, fewer than four k tiles, a batch that fills a round, no tail).
// Entry z's partials follow entry z-1's, so the workspace holds one launch's
// entries (zmax).
struct SplitSpace {
    int64_t tiles, full, rem, smax, zmax, nb;
    SplitPlan plan(int64_t split) const
    {
        if (split <= 1 || smax == 0) return SplitPlan{(int)tiles, 1, 0};
        return SplitPlan{(int)full, (int)split, (int)rem};
    }
};

SplitSpace split_space(const Problem& p, Cfg c, int64_t cus)
{
    const int64_t nb = p.batch > 1 ? p.batch : 1;
    const int64_t tiles = tile_count(p, c);
    SplitSpace s{tiles, tiles, 0, 0, nb < kMaxGridZ ? nb : kMaxGridZ, nb};
    if (is_small(c) || c == GENERIC) return s;
    const CfgInfo& ci = kCfg[c];
    const int64_t P = ci.per_cu;
    const int64_t nk = cdiv(p.k, ci.bk);
    if (nk < 4) return s;
    if (nb > 1 && tiles * nb >= P * cus) return s;
    const int64_t rem = nb > 1 ? tiles : tiles >= P * cus ? tiles % (P * cus) : tiles;
    if (rem == 0) return s;
    s.rem = rem;
    s.full = tiles - rem;
    s.smax = nk / 2 < kMaxSplit ? nk / 2 : kMaxSplit;
    return s;
}

// Bytes of split partials a plan writes (one launch's entries).
size_t split_bytes(const Problem& p, Cfg c, const SplitSpace& ss, int64_t split)
{
    const size_t elem = p.dtype == SBX_F32 ? 4 : 8;
    return (size_t)(ss.rem * split * ss.zmax) * kCfg[c].bm * kCfg[c].bn * elem;
}

double small_seconds(const Problem& p, Cfg c, int64_t cus, const SplitSpace& ss)
{
    const bool f64 = c == F64_SMALL;
    const SmallForm& f = f64 ? kSmallF64W4 : c == F32_SMALL8 ? kSmallF32W8 : kSmallF32W4;
    const int akc = !p.ta, bkc = p.tb;
    const double lay = f64 ? kSmallLayF64[akc][bkc] : kSmallLayF32[akc][bkc];
    const int64_t units = tile_count(p, c) * ss.nb;
    const double w = 2.0 * 32 * 32 * (double)p.k * lay;  // one workgroup's flops, layout-scaled
    const double lat = (double)cdiv(units, f.occ * cus) * (w / f.rs + f.wg);
    const double thr = (double)cdiv(units, cus) * (w / f.rc + f.wg);
    const double elem = f64 ? 8.0 : 4.0;
    const double bytes = ((double)p.m * p.k + (double)p.k * p.n + (double)p.m * p.n) * elem *
                         (double)ss.nb;
    const double stream = bytes / (p.batch > 1 ? kSmallBwBatch : kSmallBw);
    double t = lat > thr ? lat : thr;
    if (stream > t) t = stream;
    return f.sec + t;
}

// Modelled seconds of config c with `split` k-ranges of its tail (1: none).
double plan_seconds(const Problem& p, Cfg c, int64_t cus, const SplitSpace& ss, int64_t split,
                    bool epi)
{
    if (is_small(c)) return small_seconds(p, c, cus, ss);
    const CfgInfo& ci = kCfg[c];
    const double rate = (p.dtype == SBX_F32 ? kRateF32 : kRateF64) * cfg_eff(c);
    const double elem = p.dtype == SBX_F32 ? 4.0 : 8.0;
    const int64_t P = ci.per_cu;
    const double c_bytes = (double)ci.bm * ci.bn * elem;
    double o_tile = 0.0, o_part = 0.0;  // epilogue terms of a whole tile / a split part
    if (epi) {
        const int64_t vec_elems = 16 / (int64_t)elem;
        const bool vec = p.ldc % vec_elems == 0 && ((uintptr_t)p.C % 16) == 0;
        const double hide = P >= 3 ? 0.2 : 1.0;
        o_tile = kEpiSec * c_bytes * hide * (vec ? 1.0 : 12.0);
        o_part = kEpiSec * c_bytes * hide;
    }
    const double wk = 2.0 * ci.bm * ci.bn * (double)p.k / rate;  // a whole tile's MFMA work
    const double w = wk + o_tile + kTileSec + c_bytes / kTileStoreBw;
    const double e1 = c == F32_128x32 || c == F32_32x128 ? kE1Stream : kE1;
    if (split <= 1 || ss.smax == 0) return rounds_time(ss.tiles * ss.nb, w, P, cus, e1) + kGridSec;
    const int64_t sp = split;
    return rounds_time(ss.full * ss.nb, w, P, cus, e1) +
           rounds_time(ss.rem * sp * ss.nb, wk / (double)sp + o_part + kPartSec, P, cus, e1) +
           kGridSec + kReduceSec + (double)(ss.rem * sp * ss.nb) * c_bytes / kReduceBw;
}

// The split counts a plan may use (beyond 1, unsplit): every count to 8, then
// coarser steps, so that a pick is one of the plans that were timed.
constexpr int kSplitSet[] = {2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16, 20, 24, 28, 32};
static_assert(kMaxSplit == 32, "kSplitSet ends at kMaxSplit");

// The model's plan for config c: unsplit, or the split predicted >= 0.5 %
// faster than every smaller one (a split's partials cost memory; at 2 % the
// fp64 8192^2 x 8192 SYRK stopped at 4 parts, 7514 us, where 8-24 parts
// took 7367-7374 us).  max_ws: the most split-partial bytes a plan may use
// (the allocation-free entry point's scratch size; unlimited otherwise).
Choice model_plan(const Problem& p, Cfg c, int64_t cus, size_t max_ws, bool epi = false)
{
    const SplitSpace ss = split_space(p, c, cus);
    Choice best{c, ss.plan(1), plan_seconds(p, c, cus, ss, 1, epi)};
    for (int sp : kSplitSet) {
        if (sp > ss.smax || split_bytes(p, c, ss, sp) > max_ws) break;
        const double t = plan_seconds(p, c, cus, ss, sp, epi);
        if (t < best.seconds * 0.995) best = Choice{c, ss.plan(sp), t};
    }
    return best;
}

std::mutex g_cu_mutex;
int g_cu_count[64] = {0};

int cu_count()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> g(g_cu_mutex);
    if (!g_cu_count[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            return 256;
        g_cu_count[dev] = cus;
    }
    return g_cu_count[dev];
}

// Split-K partials and chunked-GEMV partials live in a workspace keyed by
// (device, stream): calls on one stream run in order, so they can share it.
// A stream handle is the address of the runtime's stream object, which is
// released only once the device has finished the stream's work (measured:
// hipStreamDestroy with a 68 ms kernel queued returned after 68 ms, and the
// next hipStreamCreate returned the same handle), so a handle handed out
// again finds the old kernels done.
//
// hipStreamPerThread gets no workspace: its calls run unsplit.  That handle
// names a different stream in every host thread, so its workspace would be
// the calling thread's and would change hands when the thread exits, during
// the runtime's teardown of the thread's stream.  Two such designs failed:
// ordering the handover by an event recorded on the exited thread's stream
// made the runtime report hipErrorCapturedEvent (no capture was active), and
// with the exiting thread synchronizing its stream instead, a test of six
// threads in three waves, run repeatedly in one process, aborted with
// "free(): invalid pointer" on its third run; the cause was not found.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
    // Held from handing out the workspace until the calls that use it are
    // enqueued: a split GEMM (or chunked GEMV) is two kernels, and another
    // host thread's call on the same stream must not land between them and
    // overwrite the partials the second kernel is about to read.
    std::mutex launch_mu;
};

struct WsKey {
    int dev;
    hipStream_t stream;
    bool operator<(const WsKey& o) const
    {
        if (dev != o.dev) return dev < o.dev;
        return stream < o.stream;
    }
};

std::mutex g_ws_mutex;
// never destroyed: freeing device memory during process teardown is unsafe
std::map<WsKey, Workspace*>* g_ws = new std::map<WsKey, Workspace*>();

// A workspace of at least `bytes` for `stream`, locked for the caller's
// launches until release (ptr null if there is none: hipStreamPerThread, or
// the allocation failed).  A workspace that is outgrown is retired, not
// freed: kernels enqueued earlier may not have run yet.  Growth at least
// doubles, so the retired buffers add up to less than the live one.  A
// failed runtime call here leaves its error as the thread's last error,
// which the launch check after the caller's kernels would report: since the
// caller handles the failure (it runs unsplit), that error is consumed.
struct WorkspaceLease {
    void* ptr = nullptr;
    std::unique_lock<std::mutex> lock;

    bool acquire(hipStream_t s, size_t bytes)
    {
        if (s == hipStreamPerThread) return false;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return failed();
        const WsKey key{dev, s};
        Workspace* ws;
        {
            std::lock_guard<std::mutex> g(g_ws_mutex);
            Workspace*& slot = (*g_ws)[key];
            if (!slot) slot = new Workspace();
            ws = slot;
        }
        lock = std::unique_lock<std::mutex>(ws->launch_mu);
        if (ws->bytes < bytes) {
            size_t nb = bytes < ((size_t)32 << 20) ? ((size_t)32 << 20) : bytes;
            if (nb < 2 * ws->bytes) nb = 2 * ws->bytes;
            void* p = nullptr;
            if (hipMalloc(&p, nb) != hipSuccess) return failed();  // the old buffer stays
            ws->base = p;
            ws->bytes = nb;
        }
        ptr = ws->base;
        return true;
    }

    bool failed()
    {
        (void)hipGetLastError();
        release();
        return false;
    }

    // Let the next caller in (after the caller's launches are enqueued).
    void release()
    {
        if (lock.owns_lock()) lock.unlock();
    }
    ~WorkspaceLease() { release(); }
};

hipError_t launch_cfg(Cfg cfg, GemmArgs<float>& a, bool akc, bool bkc, const Problem& p,
                      int nb, hipStream_t s)
{
    switch (cfg) {
    case F32_256x256:
        return launch_mfma<float, 256, 256, 32, 4, 2, 1, 2>(a, akc, bkc, nb, s);
    case F32_256x128:
        return launch_mfma<float, 256, 128, 16, 4, 1, 2, 2>(a, akc, bkc, nb, s);
    case F32_128x128:
        return launch_mfma<float, 128, 128, 16, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F32_128x128_O3:
        return launch_mfma<float, 128, 128, 16, 2, 2, 2, 3>(a, akc, bkc, nb, s);
    case F32_128x64:
        return launch_mfma<float, 128, 64, 32, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F32_256x64:
        return launch_mfma<float, 256, 64, 32, 8, 1, 2, 2, 1>(a, akc, bkc, nb, s);
    case F32_256x48:
        return launch_mfma<float, 256, 64, 32, 8, 1, 2, 2, 1, 48>(a, akc, bkc, nb, s);
    case F32_64x128:
        return launch_mfma<float, 64, 128, 32, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F32_64x256:
        return launch_mfma<float, 64, 256, 32, 1, 8, 2, 2, 1>(a, akc, bkc, nb, s);
    case F32_48x256:
        return launch_mfma<float, 64, 256, 32, 1, 8, 2, 2, 1, 256, 48>(a, akc, bkc, nb, s);
    case F32_128x32:
        return launch_mfma<float, 128, 32, 32, 4, 1, 2, 2, 1>(a, akc, bkc, nb, s);
    case F32_32x128:
        return launch_mfma<float, 32, 128, 32, 1, 4, 2, 2, 1>(a, akc, bkc, nb, s);
    case F32_64x64:
        return launch_mfma<float, 64, 64, 32, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F32_SMALL:
        return launch_small(a, akc, bkc, nb, s, 4);
    case F32_SMALL8:
        return launch_small(a, akc, bkc, nb, s, 8);
    default:
        a.tiles_m = (int)cdiv(p.m, 64);
        a.tiles_n = (int)cdiv(p.n, 64);
        return launch_generic<float>(a, p.ta, p.tb, nb, s);
    }
}

hipError_t launch_cfg(Cfg cfg, GemmArgs<double>& a, bool akc, bool bkc, const Problem& p,
                      int nb, hipStream_t s)
{
    switch (cfg) {
    case F64_128x128:
        return launch_mfma<double, 128, 128, 16, 2, 2, 1, 2>(a, akc, bkc, nb, s);
    case F64_128x64:
        return launch_mfma<double, 128, 64, 16, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F64_64x128:
        return launch_mfma<double, 64, 128, 16, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F64_64x64:
        return launch_mfma<double, 64, 64, 16, 2, 2, 2, 2>(a, akc, bkc, nb, s);
    case F64_SMALL:
        return launch_small(a, akc, bkc, nb, s, 4);
    default:
        a.tiles_m = (int)cdiv(p.m, 64);
        a.tiles_n = (int)cdiv(p.n, 64);
        return launch_generic<double>(a, p.ta, p.tb, nb, s);
    }
}

// The operand whose loads go non-temporal (0 none, 1 A, 2 B).  A grid one
// tile column wide reads each element of A exactly once (one tile row: B).
// When that operand is also larger than the 256 MB last-level cache, no
// cache can keep it from one call to the next, and loading it non-temporal
// leaves the caches to the other operand (bit-identical; interleaved
// timings): 65536 x 64 x 4096 (1 GiB) 271.0-271.8 -> 265.1-265.7 us,
// 131072 x 48 x 1024 (512 MiB) +2.4-4.4 %.  A smaller one keeps the default
// policy, so repeated calls find it in that cache (100000 x 63 x 515,
// 206 MB: 9 % slower non-temporal).
constexpr int64_t kStreamBytes = (int64_t)256 << 20;
int stream_operand(const Problem& p, int tiles_m, int tiles_n)
{
    const int64_t elem = p.dtype == SBX_F32 ? 4 : 8;
    const int64_t copies = p.batch > 1 ? p.batch : 1;
    if (tiles_n == 1) {
        const int64_t rows = p.ta ? p.k : p.m, cols = p.ta ? p.m : p.k;
        const int64_t per = ((rows - 1) * p.lda + cols) * elem;
        if ((p.str_a || p.table ? copies : 1) * per > kStreamBytes) return 1;
    }
    if (tiles_m == 1) {
        const int64_t rows = p.tb ? p.n : p.k, cols = p.tb ? p.k : p.n;
        const int64_t per = ((rows - 1) * p.ldb + cols) * elem;
        if ((p.str_b || p.table ? copies : 1) * per > kStreamBytes) return 2;
    }
    return 0;
}

#ifdef SBX_PROBE
// Probe build: the timestamp ring that sbx_probe_set installs, and the slot of
// the next GEMM dispatch.
static_assert(SBX_PROBE_POINTS == kStampPoints, "probe header and kernels agree");
std::mutex g_probe_mu;
unsigned long long* g_probe_buf = nullptr;
int64_t g_probe_blocks = 0, g_probe_ring = 0, g_probe_count = 0;

template <typename T>
void probe_assign(GemmArgs<T>& a)
{
    std::lock_guard<std::mutex> g(g_probe_mu);
    if (!g_probe_buf) {
        a.stamps = nullptr;
        a.stamp_blocks = 0;
        return;
    }
    a.stamps = g_probe_buf + (size_t)(g_probe_count++ % g_probe_ring) * (size_t)g_probe_blocks *
                                 kStampPoints * 2;
    a.stamp_blocks = (int)g_probe_blocks;
}
#endif

// A caller-provided split workspace: the allocation-free entry point's
// per-device scratch.  `launch_mu` plays the part of Workspace::launch_mu:
// it is held from handing out the scratch until the split kernels are
// enqueued, so another host thread's call (on the same stream or not) never
// lands between one call's partial writes and their reduction.
struct FixedScratch {
    void* ptr;
    size_t bytes;
    std::mutex* launch_mu;
};

// A plan the caller names (sbx_gemm_ex_plan): a tile config and the number
// of k-ranges its tail is cut into (1: unsplit).
struct ForcedPlan {
    Cfg cfg;
    int split;
};

// Element type a config computes in; -1 for the generic kernel (both).
int cfg_dtype(Cfg c)
{
    if (c == GENERIC) return -1;
    return strstr(kCfg[c].name, "_f64_") ? SBX_F64 : SBX_F32;
}

// "<config name>" or "<config name>+splitk<s>": the names sbx_gemm_select
// reports and sbx_gemm_ex_plan accepts.
void plan_name(Cfg c, int split, char* name, size_t cap)
{
    if (split > 1)
        snprintf(name, cap, "%s+splitk%d", kCfg[c].name, split);
    else
        snprintf(name, cap, "%s", kCfg[c].name);
}

bool parse_plan(const char* name, ForcedPlan* out)
{
    if (!name) return false;
    const char* plus = strstr(name, "+splitk");
    const size_t len = plus ? (size_t)(plus - name) : strlen(name);
    int split = 1;
    if (plus) {
        char* end = nullptr;
        const long v = strtol(plus + 7, &end, 10);
        if (end == plus + 7 || *end != '\0' || v < 2 || v > kMaxSplit) return false;
        split = (int)v;
    }
    for (int c = 0; c <= GENERIC; ++c)
        if (strlen(kCfg[c].name) == len && strncmp(kCfg[c].name, name, len) == 0) {
            *out = ForcedPlan{(Cfg)c, split};
            return true;
        }
    return false;
}

// The heuristics' last picks on this host thread.  A pick depends only on
// what the key holds (the problem's shape, transposes and leading
// dimensions, C's 16-byte alignment, whether a grouped table is used, the
// algo, the workspace limit and the device), so a repeated call -- a serving
// loop, a benchmark -- skips the model, about 2 us of host time per call.
struct PlanKey {
    int dev, dtype, algo, uplo;
    bool ta, tb, c16, table;
    int64_t m, n, k, lda, ldb, ldc, batch;
    size_t max_ws;
    bool operator==(const PlanKey& o) const
    {
        return dev == o.dev && dtype == o.dtype && algo == o.algo && uplo == o.uplo &&
               ta == o.ta && tb == o.tb && c16 == o.c16 && table == o.table && m == o.m &&
               n == o.n && k == o.k && lda == o.lda && ldb == o.ldb && ldc == o.ldc &&
               batch == o.batch && max_ws == o.max_ws;
    }
};

PlanKey plan_key(const Problem& p, int algo, size_t max_ws)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    return PlanKey{dev,   p.dtype, algo,  p.uplo, p.ta,  p.tb,  ((uintptr_t)p.C % 16) == 0,
                   p.table != nullptr, p.m, p.n, p.k, p.lda, p.ldb, p.ldc, p.batch, max_ws};
}

struct PlanCache {
    static constexpr int kSlots = 8;
    PlanKey key[kSlots];
    Cfg cfg[kSlots];
    SplitPlan sp[kSlots];
    int used = 0, next = 0;

    bool find(const PlanKey& k, Cfg* c, SplitPlan* s) const
    {
        for (int i = 0; i < used; ++i)
            if (key[i] == k) {
                *c = cfg[i];
                *s = sp[i];
                return true;
            }
        return false;
    }
    void put(const PlanKey& k, Cfg c, SplitPlan s)
    {
        key[next] = k;
        cfg[next] = c;
        sp[next] = s;
        next = (next + 1) % kSlots;
        if (used < kSlots) ++used;
    }
};
thread_local PlanCache g_plan_cache;

// fixed: the caller's split workspace; null: the stream's cached one.
// forced: run this plan instead of the model's (SBX_UNSUPPORTED if the
// problem cannot use it).
template <typename T>
int run(const Problem& p, T alpha, T beta, int algo, hipStream_t stream, Cfg* chosen,
        SplitPlan* chosen_split, const FixedScratch* fixed = nullptr,
        const ForcedPlan* forced = nullptr)
{
    if (p.m == 0 || p.n == 0 || p.batch == 0) return SBX_OK;
    const bool quick = alpha == (T)0 || p.k == 0;
    Cfg cfg = GENERIC;
    SplitPlan sp{0, 1, 0};
    if (forced) {
        const int dt = cfg_dtype(forced->cfg);
        if ((dt >= 0 && dt != p.dtype) || p.table) return SBX_UNSUPPORTED;
        // a triangle takes only the square tile configs its candidates list
        if (p.uplo && forced->cfg != F32_256x256 && forced->cfg != F32_128x128 &&
            forced->cfg != F32_128x128_O3 && forced->cfg != F64_128x128)
            return SBX_UNSUPPORTED;
        if (forced->cfg != GENERIC && !mfma_feasible(p, forced->cfg)) return SBX_UNSUPPORTED;
        const SplitSpace ss = split_space(p, forced->cfg, cu_count());
        if (forced->split > 1 && forced->split > ss.smax) return SBX_UNSUPPORTED;
        cfg = forced->cfg;
        sp = ss.plan(forced->split);
    } else if (algo != SBX_ALGO_GENERIC) {
        // no workspace for hipStreamPerThread: plan unsplit
        const size_t max_ws = fixed ? fixed->bytes : stream == hipStreamPerThread ? 0 : SIZE_MAX;
        const PlanKey key = plan_key(p, algo, max_ws);
        if (!g_plan_cache.find(key, &cfg, &sp)) {
            Cfg cands[kMaxCands];
            const int64_t cus = cu_count();
            bool large = false;
            const int nc = candidate_cfgs(p.dtype, p.m, p.n, p.uplo, cus, cands, &large);
            bool any = false;
            Choice best{GENERIC, SplitPlan{0, 1, 0}, 0.0};
            for (int i = 0; i < nc; ++i) {
                if (!mfma_feasible(p, cands[i])) continue;
                const bool small = is_small(cands[i]);
                if (algo == SBX_ALGO_MFMA_TILE && small) continue;
                if (algo == SBX_ALGO_MFMA_SMALL && !small) continue;
                const Choice c = model_plan(p, cands[i], cus, max_ws, large);
                if (!any || c.seconds < best.seconds) best = c;  // ties keep the earlier one
                any = true;
            }
            if (!any && algo != SBX_ALGO_AUTO) return SBX_UNSUPPORTED;
            if (any) {
                cfg = best.cfg;
                sp = best.sp;
            }
            g_plan_cache.put(key, cfg, sp);
        }
    }
    const CfgInfo& info = kCfg[cfg];
    const int64_t tiles = tile_count(p, cfg);
    if (cfg == GENERIC || quick) sp = SplitPlan{(int)tiles, 1, 0};
    if (chosen) *chosen = cfg;
    if (chosen_split) *chosen_split = sp;
    if (stream == (hipStream_t)-1) return SBX_OK;  // selection only
    void* ws = nullptr;
    WorkspaceLease lease;  // held until both split kernels are enqueued
    std::unique_lock<std::mutex> scratch_lock;  // the same, for the fixed scratch
    // one launch's batch entries (at most kMaxGridZ) each hold their partials
    const int64_t zmax = p.batch < 1 ? 1 : p.batch < kMaxGridZ ? p.batch : kMaxGridZ;
    const size_t ws_bytes = (size_t)sp.rem * sp.split * info.bm * info.bn * sizeof(T) * (size_t)zmax;
    if (sp.split > 1 && fixed) {
        // the planner keeps every split's partials within fixed->bytes; a plan
        // that did not fit would be refused here, never written past the end
        if (ws_bytes > fixed->bytes) return SBX_UNSUPPORTED;
        scratch_lock = std::unique_lock<std::mutex>(*fixed->launch_mu);
        ws = fixed->ptr;
    } else if (sp.split > 1) {
        if (lease.acquire(stream, ws_bytes))
            ws = lease.ptr;
        else
            sp = SplitPlan{(int)tiles, 1, 0};  // no memory: run unsplit
    }

    for (int64_t b0 = 0; b0 < p.batch; b0 += kMaxGridZ) {
        const int nb = (int)((p.batch - b0) < kMaxGridZ ? (p.batch - b0) : kMaxGridZ);
        hipError_t e;
        if (quick) {
            e = launch_scale<T>((T*)p.C + b0 * p.str_c, p.ldc, p.str_c, p.m, p.n, beta, p.relu,
                                p.uplo, nb, stream, p.table ? p.table + 3 * b0 : nullptr);
        } else {
            GemmArgs<T> a;
            a.A = (const T*)p.A + b0 * p.str_a;
            a.B = (const T*)p.B + b0 * p.str_b;
            a.C = (T*)p.C + b0 * p.str_c;
            a.lda = p.lda; a.ldb = p.ldb; a.ldc = p.ldc;
            a.str_a = p.str_a; a.str_b = p.str_b; a.str_c = p.str_c;
            a.M = (int)p.m; a.N = (int)p.n; a.K = (int)p.k;
            a.alpha = alpha; a.beta = beta;
            const CfgInfo& ci = kCfg[cfg];
            a.tiles_m = (int)cdiv(p.m, ci.bm);
            a.tiles_n = (int)cdiv(p.n, ci.bn);
            // GROUP_M: the height of the tile-column walk.  An XCD's 64
            // resident 256x128 workgroups then cover 4 x 16 tiles (1024 rows
            // of A, 2048 columns of B), which fetches 2.3 GB from beyond L2
            // at 8192^3 against 3.4 GB for 8 x 8, in the same time.  The
            // fp64 128^2 tile likewise: 12.9 GB from beyond L2 at 8192^3
            // against 13.5 GB for 8 (19.3 for 2, 22.6 for 16), same time;
            // its SYRK 9.1 against 9.4 GB.
            const int gm = cfg == F32_256x128 || cfg == F64_128x128 ? 4 : 8;
            a.group_m = a.tiles_m < gm ? a.tiles_m : gm;
            a.c_vec = p.ldc % (16 / (int64_t)sizeof(T)) == 0 && (uintptr_t)a.C % 16 == 0 &&
                      (p.batch <= 1 || p.str_c % (16 / (int64_t)sizeof(T)) == 0);
            a.num_full = sp.num_full;
            a.split = sp.split;
            a.ws = (T*)ws;
            a.relu = p.relu;
            a.uplo = p.uplo;
            a.tiles = (int)tiles;
            a.table = p.table ? p.table + 3 * b0 : nullptr;
            a.table_swap = p.table_swap;
            a.stream_op = stream_operand(p, a.tiles_m, a.tiles_n);
            // the 8-wave small-problem kernel's pairs of waves take turns at
            // the higher issue priority where each CU holds one workgroup
            // and K is long (512^2 x 2048: 13.7 against 14.6 us; on grids of
            // several rounds it lost, 1024^2 x 512: 16.9 against 14.1 us)
            a.alt_prio = cfg == F32_SMALL8 && p.k >= 1024 &&
                         (int64_t)a.tiles_m * a.tiles_n * nb <= cu_count();
#ifdef SBX_PROBE
            probe_assign(a);
#endif
            // A (m x k) is k-contiguous iff not transposed, B (k x n) iff transposed
            e = launch_cfg(cfg, a, !p.ta, p.tb != 0, p, nb, stream);
        }
        if (e != hipSuccess) return SBX_HIP_ERROR;
    }
    return SBX_OK;
}

int gemm_impl(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
              int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
              int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
              void* C, int64_t ldc, int64_t str_c, int64_t batch, int algo, int epilogue,
              Cfg* chosen, SplitPlan* chosen_split, const FixedScratch* fixed = nullptr,
              const ForcedPlan* forced = nullptr, Problem* problem = nullptr)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (epilogue != SBX_EPILOGUE_NONE && epilogue != SBX_EPILOGUE_RELU) return SBX_INVALID_ARGUMENT;
    if (layout != 0 && layout != 1) return SBX_INVALID_ARGUMENT;
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return SBX_INVALID_ARGUMENT;
    if (algo < SBX_ALGO_AUTO || algo > SBX_ALGO_MFMA_SMALL) return SBX_INVALID_ARGUMENT;
    if (m < 0 || n < 0 || k < 0 || batch < 0) return SBX_INVALID_ARGUMENT;
    if (m > kMaxDim || n > kMaxDim || k > kMaxDim) return SBX_UNSUPPORTED;
    if (!alpha || !beta) return SBX_INVALID_ARGUMENT;
    if (check_ld(layout, transA, m, k, lda) || check_ld(layout, transB, k, n, ldb) ||
        check_ld(layout, false, m, n, ldc))
        return SBX_INVALID_ARGUMENT;
    if (batch > 1 && (str_a < 0 || str_b < 0 || str_c <= 0)) return SBX_INVALID_ARGUMENT;
    const size_t elem = dtype == SBX_F32 ? 4 : 8;
    const bool alpha0 = dtype == SBX_F32 ? *(const float*)alpha == 0.0f
                                         : *(const double*)alpha == 0.0;
    if (m > 0 && n > 0 && batch > 0) {
        if (!C || (uintptr_t)C % elem) return SBX_INVALID_ARGUMENT;
        if (k > 0 && !alpha0) {
            if (!A || !B || (uintptr_t)A % elem || (uintptr_t)B % elem)
                return SBX_INVALID_ARGUMENT;
        }
    }

    // Column-major C (m x n) is row-major C^T (n x m) = op(B)^T op(A)^T: swap
    // the operands and the sizes, keep each operand's own transpose flag.
    Problem p;
    p.dtype = dtype;
    if (layout == 0) {
        p.ta = transA; p.tb = transB; p.m = m; p.n = n;
        p.A = A; p.lda = lda; p.str_a = str_a;
        p.B = B; p.ldb = ldb; p.str_b = str_b;
    } else {
        p.ta = transB; p.tb = transA; p.m = n; p.n = m;
        p.A = B; p.lda = ldb; p.str_a = str_b;
        p.B = A; p.ldb = lda; p.str_b = str_a;
    }
    p.k = k; p.C = C; p.ldc = ldc; p.str_c = batch > 1 ? str_c : 0; p.batch = batch;
    p.relu = epilogue == SBX_EPILOGUE_RELU;
    p.uplo = 0;
    p.table = nullptr;
    p.table_swap = 0;
    if (batch <= 1) { p.str_a = 0; p.str_b = 0; }
    if (problem) {  // the validated problem only (plan enumeration)
        *problem = p;
        return SBX_OK;
    }

    hipStream_t s = (hipStream_t)stream;
    if (dtype == SBX_F32)
        return run<float>(p, *(const float*)alpha, *(const float*)beta, algo, s, chosen,
                          chosen_split, fixed, forced);
    return run<double>(p, *(const double*)alpha, *(const double*)beta, algo, s, chosen,
                       chosen_split, fixed, forced);
}

// Grouped GEMM: `count` problems of one shape and one set of scalars whose
// operands are scattered (a device table of A_i, B_i, C_i pointers), run as
// one batched launch -- what the task graph uses to issue runs of
// independent same-shaped GEMMs without one launch each.
int grouped_impl(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                 int64_t n, int64_t k, const void* alpha, int64_t lda, int64_t ldb,
                 const void* beta, int64_t ldc, const void* const* table, int64_t count,
                 int aligned16, int epilogue)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (epilogue != SBX_EPILOGUE_NONE && epilogue != SBX_EPILOGUE_RELU) return SBX_INVALID_ARGUMENT;
    if (layout != 0 && layout != 1) return SBX_INVALID_ARGUMENT;
    if ((transA != 0 && transA != 1) || (transB != 0 && transB != 1)) return SBX_INVALID_ARGUMENT;
    if (m < 0 || n < 0 || k < 0 || count < 0) return SBX_INVALID_ARGUMENT;
    if (m > kMaxDim || n > kMaxDim || k > kMaxDim) return SBX_UNSUPPORTED;
    if (!alpha || !beta) return SBX_INVALID_ARGUMENT;
    if (check_ld(layout, transA, m, k, lda) || check_ld(layout, transB, k, n, ldb) ||
        check_ld(layout, false, m, n, ldc))
        return SBX_INVALID_ARGUMENT;
    if (m == 0 || n == 0 || count == 0) return SBX_OK;
    if (!table || (uintptr_t)table % sizeof(void*)) return SBX_INVALID_ARGUMENT;
    // alignment stand-ins: never dereferenced, they carry the caller's promise
    const void* stand_in = (const void*)(uintptr_t)(aligned16 ? 0x1000 : 0x1004);
    Problem p;
    p.dtype = dtype;
    if (layout == 0) {
        p.ta = transA; p.tb = transB; p.m = m; p.n = n;
        p.lda = lda; p.ldb = ldb;
        p.table_swap = 0;
    } else {
        p.ta = transB; p.tb = transA; p.m = n; p.n = m;
        p.lda = ldb; p.ldb = lda;
        p.table_swap = 1;
    }
    p.A = stand_in; p.B = stand_in; p.C = const_cast<void*>(stand_in);
    p.str_a = 0; p.str_b = 0; p.str_c = 0;
    p.k = k; p.ldc = ldc; p.batch = count;
    p.relu = epilogue == SBX_EPILOGUE_RELU;
    p.uplo = 0;
    p.table = table;
    hipStream_t s = (hipStream_t)stream;
    if (dtype == SBX_F32)
        return run<float>(p, *(const float*)alpha, *(const float*)beta, SBX_ALGO_AUTO, s, nullptr,
                          nullptr);
    return run<double>(p, *(const double*)alpha, *(const double*)beta, SBX_ALGO_AUTO, s, nullptr,
                       nullptr);
}

// One line "<plan name> <predicted microseconds>" per plan the heuristics
// weigh for problem p (every candidate config, unsplit and at each split of
// kSplitSet its split space allows), the pick among them.
int write_plans(const Problem& p, char* out, size_t cap)
{
    out[0] = '\0';
    if (p.m == 0 || p.n == 0 || p.batch == 0) return SBX_OK;
    const int64_t cus = cu_count();
    Cfg cands[kMaxCands];
    bool large = false;
    const int nc = candidate_cfgs(p.dtype, p.m, p.n, p.uplo, cus, cands, &large);
    size_t used = 0;
    for (int i = 0; i < nc; ++i) {
        const Cfg c = cands[i];
        if (!mfma_feasible(p, c)) continue;
        const SplitSpace ss = split_space(p, c, cus);
        for (int j = -1; j < (int)(sizeof(kSplitSet) / sizeof(int)); ++j) {
            const int s = j < 0 ? 1 : kSplitSet[j];
            if (s > 1 && s > ss.smax) break;
            char name[96];
            plan_name(c, s, name, sizeof(name));
            const double us = plan_seconds(p, c, cus, ss, s, large) * 1e6;
            const int w = snprintf(out + used, cap - used, "%s %.3f\n", name, us);
            if (w < 0 || (size_t)w >= cap - used) {
                out[used] = '\0';
                return SBX_INVALID_ARGUMENT;  // buffer too small
            }
            used += (size_t)w;
        }
    }
    return SBX_OK;
}

// SYRK: C = alpha * op(A) op(A)^T + beta * C on one triangle of the n x n C
// (the arithmetic of oneMKL's syrk / syrk_batch, syrk.cpp:44-77), run as a
// GEMM with B = A whose tile grid covers only that triangle.  Row-major:
// trans == 0 is A (n x k) times A^T, trans == 1 is A^T A with A k x n.  A
// column-major call is the row-major one on the same memory with `upper` and
// `trans` flipped (column-major C's lower triangle is row-major C^T's upper,
// and a column-major n x k A is a row-major k x n one).
int syrk_impl(void* stream, int dtype, int layout, int upper, int trans, int64_t n, int64_t k,
              const void* alpha, const void* A, int64_t lda, int64_t str_a, const void* beta,
              void* C, int64_t ldc, int64_t str_c, int64_t batch, Cfg* chosen = nullptr,
              SplitPlan* chosen_split = nullptr, const ForcedPlan* forced = nullptr,
              Problem* problem = nullptr)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (layout != 0 && layout != 1) return SBX_INVALID_ARGUMENT;
    if ((upper != 0 && upper != 1) || (trans != 0 && trans != 1)) return SBX_INVALID_ARGUMENT;
    if (n < 0 || k < 0 || batch < 0) return SBX_INVALID_ARGUMENT;
    if (n > kMaxDim || k > kMaxDim) return SBX_UNSUPPORTED;
    if (!alpha || !beta) return SBX_INVALID_ARGUMENT;
    if (check_ld(layout, trans, n, k, lda) || check_ld(layout, false, n, n, ldc))
        return SBX_INVALID_ARGUMENT;
    if (batch > 1 && (str_a < 0 || str_c <= 0)) return SBX_INVALID_ARGUMENT;
    const size_t elem = dtype == SBX_F32 ? 4 : 8;
    const bool alpha0 = dtype == SBX_F32 ? *(const float*)alpha == 0.0f
                                         : *(const double*)alpha == 0.0;
    if (n > 0 && batch > 0) {
        if (!C || (uintptr_t)C % elem) return SBX_INVALID_ARGUMENT;
        if (k > 0 && !alpha0 && (!A || (uintptr_t)A % elem)) return SBX_INVALID_ARGUMENT;
    }
    const int up = layout == 0 ? upper : !upper;
    const int tr = layout == 0 ? trans : !trans;
    Problem p;
    p.dtype = dtype;
    p.ta = tr;
    p.tb = !tr;
    p.m = n; p.n = n; p.k = k;
    p.A = A; p.lda = lda; p.str_a = batch > 1 ? str_a : 0;
    p.B = A; p.ldb = lda; p.str_b = p.str_a;
    p.C = C; p.ldc = ldc; p.str_c = batch > 1 ? str_c : 0;
    p.batch = batch;
    p.relu = 0;
    p.uplo = up ? 2 : 1;
    p.table = nullptr;
    p.table_swap = 0;
    if (problem) {
        *problem = p;
        return SBX_OK;
    }
    hipStream_t s = (hipStream_t)stream;
    if (dtype == SBX_F32)
        return run<float>(p, *(const float*)alpha, *(const float*)beta, SBX_ALGO_AUTO, s,
                          chosen, chosen_split, nullptr, forced);
    return run<double>(p, *(const double*)alpha, *(const double*)beta, SBX_ALGO_AUTO, s,
                       chosen, chosen_split, nullptr, forced);
}

// GEMV: y = alpha * op(A) x + beta * y (oneMKL gemv, gemv.cpp:44-61), netlib
// quick returns: m == 0 or n == 0 leaves y untouched; alpha == 0 gives
// y = beta * y (zeros when beta == 0, y not read).  A column-major m x n A is
// a row-major n x m A^T, so the transpose flag flips.
template <typename T>
int gemv_run(hipStream_t stream, bool trans, int64_t rows, int64_t cols, T alpha, const T* A,
             int64_t lda, const T* x, int64_t incx, T beta, T* y, int64_t incy)
{
    const int64_t ylen = trans ? cols : rows;
    if (alpha == (T)0) {
        if (beta == (T)1) return SBX_OK;
        // y as a ylen x 1 matrix with row pitch incy
        return launch_scale<T>(y, incy, 0, ylen, 1, beta, 0, 0, 1, stream) == hipSuccess
                   ? SBX_OK : SBX_HIP_ERROR;
    }
    // 16-byte loads of A at any row alignment (the device serves unaligned
    // multi-dword loads); the row-dot form also reads x in vectors, so it
    // needs x contiguous
    const bool vec = trans || incx == 1;
    GemvPlan pl = plan_gemv<T>(trans, rows, cols, vec, cu_count());
    GemvArgs<T> a;
    a.A = A; a.x = x; a.y = y;
    a.lda = lda; a.incx = incx; a.incy = incy;
    a.rows = rows; a.cols = cols;
    a.alpha = alpha; a.beta = beta;
    a.cw = pl.cw;
    a.ws = nullptr;
    WorkspaceLease lease;  // held until the partial and finish kernels are enqueued
    if (pl.chunks > 1) {
        a.ws = lease.acquire(stream, (size_t)pl.chunks * pl.out_len * sizeof(T))
                   ? (T*)lease.ptr : nullptr;
        if (!a.ws) {  // no memory for partials: one range
            pl.chunks = 1;
            pl.cw = trans ? rows : cols;
        }
    }
    if (launch_gemv<T>(a, pl, stream) != hipSuccess) return SBX_HIP_ERROR;
    return SBX_OK;
}

int gemv_impl(void* stream, int dtype, int layout, int trans, int64_t m, int64_t n,
              const void* alpha, const void* A, int64_t lda, const void* x, int64_t incx,
              const void* beta, void* y, int64_t incy)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (layout != 0 && layout != 1) return SBX_INVALID_ARGUMENT;
    if (trans != 0 && trans != 1) return SBX_INVALID_ARGUMENT;
    if (m < 0 || n < 0) return SBX_INVALID_ARGUMENT;
    if (incx == 0 || incy == 0) return SBX_INVALID_ARGUMENT;
    if (incx < 0 || incy < 0) return SBX_UNSUPPORTED;
    if (!alpha || !beta) return SBX_INVALID_ARGUMENT;
    if (check_ld(layout, false, m, n, lda)) return SBX_INVALID_ARGUMENT;
    if (m == 0 || n == 0) return SBX_OK;
    const size_t elem = dtype == SBX_F32 ? 4 : 8;
    const bool alpha0 = dtype == SBX_F32 ? *(const float*)alpha == 0.0f
                                         : *(const double*)alpha == 0.0;
    if (!y || (uintptr_t)y % elem) return SBX_INVALID_ARGUMENT;
    if (!alpha0 && (!A || !x || (uintptr_t)A % elem || (uintptr_t)x % elem))
        return SBX_INVALID_ARGUMENT;
    const bool t = layout == 0 ? trans != 0 : trans == 0;
    const int64_t rows = layout == 0 ? m : n, cols = layout == 0 ? n : m;
    hipStream_t s = (hipStream_t)stream;
    if (dtype == SBX_F32)
        return gemv_run<float>(s, t, rows, cols, *(const float*)alpha, (const float*)A, lda,
                               (const float*)x, incx, *(const float*)beta, (float*)y, incy);
    return gemv_run<double>(s, t, rows, cols, *(const double*)alpha, (const double*)A, lda,
                            (const double*)x, incx, *(const double*)beta, (double*)y, incy);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (sbx_gemm_ex_noalloc): split-K
// partials go to this fixed array instead of the stream workspace, so that
// entry point makes no allocation.  Each device holds its own copy from the
// library's first use on it until the process ends.  In host code `scratch`
// names a host-side stand-in, not a device address: the device address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that address is ever passed to kernels.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = SBX_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size must keep partial slots aligned");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[64] = {nullptr};
// per device: held while one call enqueues the kernels that use the scratch
std::mutex g_scratch_launch_mu[64];

// The current device's scratch (address of `scratch`, its size and launch
// lock); false if the lookup fails.
bool device_scratch(FixedScratch* out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    std::lock_guard<std::mutex> g(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return false;
        g_scratch_ptr[dev] = p;
    }
    *out = FixedScratch{g_scratch_ptr[dev], kScratchBytes, &g_scratch_launch_mu[dev]};
    return true;
}

}  // namespace
}  // namespace sbx

extern "C" {

int sbx_gemm_ex(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                void* C, int64_t ldc, int64_t str_c, int64_t batch, int algo)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::gemm_impl(stream, dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a,
                          B, ldb, str_b, beta, C, ldc, str_c, batch, algo, SBX_EPILOGUE_NONE,
                          nullptr, nullptr);
}

int sbx_gemm_ex_noalloc(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                        int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                        int64_t str_a, const void* B, int64_t ldb, int64_t str_b,
                        const void* beta, void* C, int64_t ldc, int64_t str_c, int64_t batch,
                        int algo)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    sbx::FixedScratch ws;
    if (!sbx::device_scratch(&ws)) return SBX_HIP_ERROR;
    return sbx::gemm_impl(stream, dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a,
                          B, ldb, str_b, beta, C, ldc, str_c, batch, algo, SBX_EPILOGUE_NONE,
                          nullptr, nullptr, &ws);
}

int sbx_gemm_fused(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                   int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                   int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                   void* C, int64_t ldc, int64_t str_c, int64_t batch, int epilogue)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::gemm_impl(stream, dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a,
                          B, ldb, str_b, beta, C, ldc, str_c, batch, SBX_ALGO_AUTO, epilogue,
                          nullptr, nullptr);
}

int sbx_gemm_grouped(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                     int64_t n, int64_t k, const void* alpha, int64_t lda, int64_t ldb,
                     const void* beta, int64_t ldc, const void* const* table, int64_t count,
                     int aligned16, int epilogue)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::grouped_impl(stream, dtype, layout, transA, transB, m, n, k, alpha, lda, ldb,
                             beta, ldc, table, count, aligned16, epilogue);
}

int sbx_relu(void* stream, int dtype, void* x, int64_t n)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (n < 0 || (n > 0 && !x)) return SBX_INVALID_ARGUMENT;
    if ((uintptr_t)x % (dtype == SBX_F32 ? 4 : 8)) return SBX_INVALID_ARGUMENT;
    if (n == 0) return SBX_OK;
    const hipError_t e = dtype == SBX_F32
        ? sbx::launch_relu<float>((float*)x, n, (hipStream_t)stream)
        : sbx::launch_relu<double>((double*)x, n, (hipStream_t)stream);
    return e == hipSuccess ? SBX_OK : SBX_HIP_ERROR;
}

int sbx_sgemv(void* stream, int layout, int transA, int64_t m, int64_t n, float alpha,
              const float* A, int64_t lda, const float* x, int64_t incx, float beta, float* y,
              int64_t incy)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::gemv_impl(stream, SBX_F32, layout, transA, m, n, &alpha, A, lda, x, incx, &beta,
                          y, incy);
}

int sbx_dgemv(void* stream, int layout, int transA, int64_t m, int64_t n, double alpha,
              const double* A, int64_t lda, const double* x, int64_t incx, double beta,
              double* y, int64_t incy)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::gemv_impl(stream, SBX_F64, layout, transA, m, n, &alpha, A, lda, x, incx, &beta,
                          y, incy);
}

int sbx_ssyrk_strided_batched(void* stream, int layout, int upper, int trans, int64_t n,
                              int64_t k, float alpha, const float* A, int64_t lda, int64_t str_a,
                              float beta, float* C, int64_t ldc, int64_t str_c, int64_t batch)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::syrk_impl(stream, SBX_F32, layout, upper, trans, n, k, &alpha, A, lda, str_a,
                          &beta, C, ldc, str_c, batch);
}

int sbx_dsyrk_strided_batched(void* stream, int layout, int upper, int trans, int64_t n,
                              int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    return sbx::syrk_impl(stream, SBX_F64, layout, upper, trans, n, k, &alpha, A, lda, str_a,
                          &beta, C, ldc, str_c, batch);
}

int sbx_ssyrk(void* stream, int layout, int upper, int trans, int64_t n, int64_t k, float alpha,
              const float* A, int64_t lda, float beta, float* C, int64_t ldc)
{
    return sbx_ssyrk_strided_batched(stream, layout, upper, trans, n, k, alpha, A, lda, 0, beta,
                                     C, ldc, 0, 1);
}

int sbx_dsyrk(void* stream, int layout, int upper, int trans, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, double beta, double* C, int64_t ldc)
{
    return sbx_dsyrk_strided_batched(stream, layout, upper, trans, n, k, alpha, A, lda, 0, beta,
                                     C, ldc, 0, 1);
}

int sbx_sgemm(void* stream, int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
              float* C, int64_t ldc)
{
    return sbx_gemm_ex(stream, SBX_F32, layout, transA, transB, m, n, k, &alpha, A, lda, 0, B,
                       ldb, 0, &beta, C, ldc, 0, 1, SBX_ALGO_AUTO);
}

int sbx_dgemm(void* stream, int layout, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double* A, int64_t lda, const double* B, int64_t ldb,
              double beta, double* C, int64_t ldc)
{
    return sbx_gemm_ex(stream, SBX_F64, layout, transA, transB, m, n, k, &alpha, A, lda, 0, B,
                       ldb, 0, &beta, C, ldc, 0, 1, SBX_ALGO_AUTO);
}

int sbx_sgemm_strided_batched(void* stream, int layout, int transA, int transB, int64_t m,
                              int64_t n, int64_t k, float alpha, const float* A, int64_t lda,
                              int64_t str_a, const float* B, int64_t ldb, int64_t str_b,
                              float beta, float* C, int64_t ldc, int64_t str_c, int64_t batch)
{
    return sbx_gemm_ex(stream, SBX_F32, layout, transA, transB, m, n, k, &alpha, A, lda, str_a,
                       B, ldb, str_b, &beta, C, ldc, str_c, batch, SBX_ALGO_AUTO);
}

int sbx_dgemm_strided_batched(void* stream, int layout, int transA, int transB, int64_t m,
                              int64_t n, int64_t k, double alpha, const double* A, int64_t lda,
                              int64_t str_a, const double* B, int64_t ldb, int64_t str_b,
                              double beta, double* C, int64_t ldc, int64_t str_c,
                              int64_t batch)
{
    return sbx_gemm_ex(stream, SBX_F64, layout, transA, transB, m, n, k, &alpha, A, lda, str_a,
                       B, ldb, str_b, &beta, C, ldc, str_c, batch, SBX_ALGO_AUTO);
}

int sbx_gemm_select(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                    int64_t k, int64_t lda, int64_t ldb, int64_t ldc, char* name, size_t cap)
{
    return sbx_gemm_select_batched(dtype, layout, transA, transB, m, n, k, lda, ldb, ldc, 1, name,
                                   cap);
}

int sbx_gemm_select_batched(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                            int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch,
                            char* name, size_t cap)
{
    if (!name || cap == 0) return SBX_INVALID_ARGUMENT;
    if (batch < 1) return SBX_INVALID_ARGUMENT;
    // packed entries: each stride is its operand's stored extent
    const int64_t rows_a = (layout == 0) == !transA ? m : k;
    const int64_t rows_b = (layout == 0) == !transB ? k : n;
    const int64_t rows_c = layout == 0 ? m : n;
    const int64_t str_a = rows_a * lda, str_b = rows_b * ldb, str_c = rows_c * ldc;
    static const float one_f = 1.0f;
    static const double one_d = 1.0;
    const void* one = dtype == SBX_F64 ? (const void*)&one_d : (const void*)&one_f;
    // 16-byte aligned stand-in addresses: selection never dereferences them.
    const void* fake = (const void*)(uintptr_t)0x1000;
    sbx::Cfg cfg = sbx::GENERIC;
    sbx::SplitPlan sp{0, 1, 0};
    int st = sbx::gemm_impl((void*)-1, dtype, layout, transA, transB, m, n, k, one, fake, lda,
                            str_a, fake, ldb, str_b, one, (void*)fake, ldc, str_c, batch,
                            SBX_ALGO_AUTO, SBX_EPILOGUE_NONE, &cfg, &sp);
    if (st != SBX_OK) return st;
    sbx::plan_name(cfg, sp.split, name, cap);
    return SBX_OK;
}

int sbx_gemm_plans(int dtype, int layout, int transA, int transB, int64_t m, int64_t n,
                   int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch, char* out,
                   size_t cap)
{
    if (!out || cap == 0) return SBX_INVALID_ARGUMENT;
    if (batch < 1) return SBX_INVALID_ARGUMENT;
    const int64_t rows_a = (layout == 0) == !transA ? m : k;
    const int64_t rows_b = (layout == 0) == !transB ? k : n;
    const int64_t rows_c = layout == 0 ? m : n;
    static const float one_f = 1.0f;
    static const double one_d = 1.0;
    const void* one = dtype == SBX_F64 ? (const void*)&one_d : (const void*)&one_f;
    const void* fake = (const void*)(uintptr_t)0x1000;
    sbx::Problem p;
    int st = sbx::gemm_impl((void*)-1, dtype, layout, transA, transB, m, n, k, one, fake, lda,
                            rows_a * lda, fake, ldb, rows_b * ldb, one, (void*)fake, ldc,
                            rows_c * ldc, batch, SBX_ALGO_AUTO, SBX_EPILOGUE_NONE, nullptr,
                            nullptr, nullptr, nullptr, &p);
    if (st != SBX_OK) return st;
    return sbx::write_plans(p, out, cap);
}

int sbx_gemm_ex_plan(void* stream, int dtype, int layout, int transA, int transB, int64_t m,
                     int64_t n, int64_t k, const void* alpha, const void* A, int64_t lda,
                     int64_t str_a, const void* B, int64_t ldb, int64_t str_b, const void* beta,
                     void* C, int64_t ldc, int64_t str_c, int64_t batch, const char* plan)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    sbx::ForcedPlan fp;
    if (!sbx::parse_plan(plan, &fp)) return SBX_INVALID_ARGUMENT;
    return sbx::gemm_impl(stream, dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a,
                          B, ldb, str_b, beta, C, ldc, str_c, batch, SBX_ALGO_AUTO,
                          SBX_EPILOGUE_NONE, nullptr, nullptr, nullptr, &fp);
}

int sbx_syrk_select(int dtype, int layout, int upper, int trans, int64_t n, int64_t k,
                    int64_t lda, int64_t ldc, char* name, size_t cap)
{
    if (!name || cap == 0) return SBX_INVALID_ARGUMENT;
    static const float one_f = 1.0f;
    static const double one_d = 1.0;
    const void* one = dtype == SBX_F64 ? (const void*)&one_d : (const void*)&one_f;
    const void* fake = (const void*)(uintptr_t)0x1000;
    sbx::Cfg cfg = sbx::GENERIC;
    sbx::SplitPlan sp{0, 1, 0};
    int st = sbx::syrk_impl((void*)-1, dtype, layout, upper, trans, n, k, one, fake, lda, 0, one,
                            (void*)fake, ldc, 0, 1, &cfg, &sp);
    if (st != SBX_OK) return st;
    sbx::plan_name(cfg, sp.split, name, cap);
    return SBX_OK;
}

int sbx_syrk_plans(int dtype, int layout, int upper, int trans, int64_t n, int64_t k,
                   int64_t lda, int64_t ldc, char* out, size_t cap)
{
    if (!out || cap == 0) return SBX_INVALID_ARGUMENT;
    static const float one_f = 1.0f;
    static const double one_d = 1.0;
    const void* one = dtype == SBX_F64 ? (const void*)&one_d : (const void*)&one_f;
    const void* fake = (const void*)(uintptr_t)0x1000;
    sbx::Problem p;
    const int st = sbx::syrk_impl((void*)-1, dtype, layout, upper, trans, n, k, one, fake, lda, 0,
                                  one, (void*)fake, ldc, 0, 1, nullptr, nullptr, nullptr, &p);
    if (st != SBX_OK) return st;
    return sbx::write_plans(p, out, cap);
}

int sbx_syrk_ex_plan(void* stream, int dtype, int layout, int upper, int trans, int64_t n,
                     int64_t k, const void* alpha, const void* A, int64_t lda, int64_t str_a,
                     const void* beta, void* C, int64_t ldc, int64_t str_c, int64_t batch,
                     const char* plan)
{
    if (stream == (void*)-1) return SBX_INVALID_ARGUMENT;
    sbx::ForcedPlan fp;
    if (!sbx::parse_plan(plan, &fp)) return SBX_INVALID_ARGUMENT;
    return sbx::syrk_impl(stream, dtype, layout, upper, trans, n, k, alpha, A, lda, str_a, beta, C,
                          ldc, str_c, batch, nullptr, nullptr, &fp);
}

const char* sbx_status_string(int status)
{
    switch (status) {
    case SBX_OK: return "success";
    case SBX_INVALID_ARGUMENT: return "invalid argument";
    case SBX_UNSUPPORTED: return "unsupported data type or shape";
    case SBX_HIP_ERROR: return "HIP runtime error";
    default: return "unknown status";
    }
}

int sbx_fill_uniform(void* stream, int dtype, void* out, int64_t n, uint64_t seed,
                     uint32_t stream_id)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (n < 0 || (n > 0 && !out)) return SBX_INVALID_ARGUMENT;
    if (n == 0) return SBX_OK;
    return sbx::launch_fill_uniform(dtype, out, n, seed, stream_id, (hipStream_t)stream) ==
                   hipSuccess
               ? SBX_OK
               : SBX_HIP_ERROR;
}

int sbx_fill_normal(void* stream, int dtype, void* out, int64_t n, uint64_t seed,
                    uint32_t stream_id, double scale)
{
    if (dtype != SBX_F32 && dtype != SBX_F64) return SBX_UNSUPPORTED;
    if (n < 0 || (n > 0 && !out)) return SBX_INVALID_ARGUMENT;
    if (n == 0) return SBX_OK;
    return sbx::launch_fill_normal(dtype, out, n, seed, stream_id, scale, (hipStream_t)stream) ==
                   hipSuccess
               ? SBX_OK
               : SBX_HIP_ERROR;
}

const char* sbx_version(void) { return "sushiblas_amd 0.1.0 (gfx950)"; }

#ifdef SBX_PROBE
int sbx_probe_set(void* buf, int64_t blocks, int64_t ring)
{
    if (buf && (blocks <= 0 || blocks > (int64_t)1 << 20 || ring <= 0 ||
                (uintptr_t)buf % sizeof(unsigned long long)))
        return SBX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> g(sbx::g_probe_mu);
    sbx::g_probe_buf = static_cast<unsigned long long*>(buf);
    sbx::g_probe_blocks = buf ? blocks : 0;
    sbx::g_probe_ring = buf ? ring : 0;
    sbx::g_probe_count = 0;
    return SBX_OK;
}

int64_t sbx_probe_dispatches(void)
{
    std::lock_guard<std::mutex> g(sbx::g_probe_mu);
    return sbx::g_probe_count;
}

int64_t sbx_probe_wall_clock_khz(void)
{
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
        return 0;
    return khz;
}
#endif

}  // extern "C"
