// C ABI of the gfx950 skinny decode GEMM (declared in include/krk_gemm.h).
//
// Host responsibilities: argument validation (the reference's launchers raise
// ValueError for these, engine/kernels/gateup64.py:63-74,
// engine/kernels/gemm.py:253-254), the static shape -> configuration table
// that replaces the warm-up pickers (engine/kernels/gemm.py:417-498), and
// stream-ordered kernel launches.  Nothing here allocates, synchronises or
// touches device memory from the host, so every call is graph-capturable.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdlib.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <utility>

#include "krk_gemm.h"
#include "krk_mfma.h"
#include "krk_mfma_lds.h"
#include "krk_norm.h"
#include "krk_select.h"
#include "krk_slice.h"
#include "krk_stream.h"
#include "krk_valu.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

constexpr int kMaxRowsPerLaunch = 64;
constexpr int kValuMaxRows = 8;
constexpr int kCuCount = 256;  // MI355X: 8 XCDs x 32 CUs
// LDS per workgroup this build plans for (the portable 64 KB), and what the
// kernels' static __shared__ variables take beside the dynamic reduction area.
constexpr size_t kLdsBudget = 65536;
constexpr size_t kLdsReserve = 1024;

inline int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int cdiv_c(int a, int b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool valid_epilogue(int e) { return e == KRK_EPILOGUE_NONE || e == KRK_EPILOGUE_SILU_MUL; }

int check_shape(int M, int N, int K, int epilogue) {
    if (M < 1 || N < 1 || K < 8) return fail(KRK_ERR_INVALID, "shape M=%d N=%d K=%d: need M >= 1, N >= 1, K >= 8", M, N, K);
    if (K % 8) return fail(KRK_ERR_INVALID, "K=%d must be a multiple of 8 (16-byte rows)", K);
    if (!valid_epilogue(epilogue)) return fail(KRK_ERR_INVALID, "unknown epilogue %d", epilogue);
    if (epilogue == KRK_EPILOGUE_SILU_MUL && (N % 2)) return fail(KRK_ERR_INVALID, "SILU_MUL needs an even N (gate rows then up rows), got N=%d", N);
    return KRK_OK;
}

// Channels of output per block and block count for a configuration.
struct Geometry {
    int Mc;       // rows per launch
    int Nout;     // output columns
    int cb;       // output channels per block
    int nblocks;  // blocks along N
};

Geometry geometry(int M, int N, int epilogue, const krk_gemm_config& c) {
    Geometry g;
    g.Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    const bool silu = epilogue == KRK_EPILOGUE_SILU_MUL;
    g.Nout = silu ? N / 2 : N;
    if (c.kernel == KRK_KERNEL_VALU) {
        g.cb = c.waves * (silu ? c.n_tiles / 2 : c.n_tiles);  // n_tiles W rows per wave
    } else if (c.kernel == KRK_KERNEL_STREAM) {
        g.cb = silu ? 8 : 16;  // one 16-row tile: 16 channels, or 8 gate + 8 up rows
    } else if ((c.kernel == KRK_KERNEL_MFMA_LDS || c.kernel == KRK_KERNEL_SLICE) && c.channels > 0) {
        g.cb = c.channels;
    } else {
        g.cb = 16 * (silu ? c.n_tiles / 2 : c.n_tiles);
    }
    g.nblocks = cdiv(g.Nout, g.cb);
    return g;
}

// SLICE: rows a launch may hold (two 16-row x tiles), most channels per
// block (two weight tiles), and the instantiated variants: k per chunk KC,
// weight tiles NT, weight / x groups per chunk NGV / XGV (rows of RG =
// 1024 / (2·KC) each) and chunks in flight per wave D.  128-k chunks serve up
// to 16 channels and 16 rows with 2 in flight (measured fastest for o and
// down at M <= 12); 64-k chunks up to 32 of each.  Every wave's ring of D
// slots of NGV + XGV KB fits the 160 KB of LDS.
constexpr int kSliceMaxRows = 32;
constexpr int kSliceMaxChannels = 32;
constexpr bool slice_inst(int KC, int NT, int NGV, int XGV, int D) {
    if (KC != 64 && KC != 128) return false;
    if (D < 2 || D > 3 || XGV < 1 || NGV < 1) return false;
    if ((size_t)krk::kSliceWaves * D * (NGV + XGV) * krk::kSliceGroup + kLdsReserve > 163840) return false;
    if (KC == 64) return XGV <= 4 && (NT == 1 ? NGV <= 2 : (NT == 2 && NGV >= 3 && NGV <= 4));
    return NT == 1 && NGV <= 4 && XGV <= 4 && D == 2;
}
struct SliceShape {
    int NT, NGV, XGV, MT;
};
inline SliceShape slice_shape(int KC, int cb, int Mc) {
    const int rg = krk::slice_rg(KC);
    SliceShape v;
    v.NT = cdiv(cb, 16);
    v.NGV = cdiv(cb, rg);
    v.XGV = cdiv(Mc, rg);
    v.MT = cdiv(v.XGV * rg, 16);
    return v;
}

// The dispatch table.  Every projection is HBM-bound (arithmetic intensity is
// about M flop/byte), so the table only decides how the weight stream is cut.
// Entries for the five Qwen3-4B projections were chosen by timing every
// configuration on an MI355X (graph replay over 24 distinct weight copies),
// then checked against the warm-up tuner's search over krk_gemm_candidates
// (entries it beat by 3% or more were replaced); other shapes use the rule in
// auto_config below.
struct TableEntry {
    int N, K, epilogue, m_lo, m_hi;
    krk_gemm_config cfg;  // m_tiles 0: derived from M
};
constexpr krk_gemm_config kcfg(int kernel, int n_tiles, int unroll, int waves, int splits, int k_chunk = 0,
                               int channels = 0, int x_preload = 0) {
    return krk_gemm_config{kernel, 0, n_tiles, unroll, waves, splits, k_chunk, 0, channels, x_preload};
}
// VALU entries: n_tiles = W rows per wave, unroll = 512-k blocks in flight per
// row (0: enough to cover a split's K range in one pass).  MFMA_LDS entries: unroll = stages in
// flight, k_chunk 0 = 512 where it fits, channels 0 = all of the tiles' channels.
const TableEntry kTable[] = {
    // qkv 2560 -> 6144
    {6144, 2560, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 1, 0, 8, 1)},
    {6144, 2560, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 0, 4, 1)},
    {6144, 2560, KRK_EPILOGUE_NONE, 3, 4, kcfg(KRK_KERNEL_VALU, 1, 0, 8, 1)},
    // Whole K per block.  M = 5-24: the wave-sliced kernel on 256 blocks of 24
    // channels, 64-k chunks, 2 in flight per wave (M = 8: 7.5 against 8.3 us,
    // M = 20: 8.9 against 9.6 us for the LDS-staged kernel); M = 25-32: x held
    // in registers for the whole K, 192 blocks of 32 channels, 3 stages in
    // flight; M = 33-64: 256 blocks of 24 channels, one per CU, x staged per
    // 256-k stage.
    {6144, 2560, KRK_EPILOGUE_NONE, 5, 24, kcfg(KRK_KERNEL_SLICE, 0, 2, 0, 1, 64, 24)},
    {6144, 2560, KRK_EPILOGUE_NONE, 25, 32, kcfg(KRK_KERNEL_MFMA_LDS, 2, 3, 0, 1, 512, 32, 2)},
    {6144, 2560, KRK_EPILOGUE_NONE, 33, 64, kcfg(KRK_KERNEL_MFMA_LDS, 2, 3, 0, 1, 256, 24)},
    // o_proj 4096 -> 2560
    // 5-wave workgroups: 256 of 2 rows per wave at M <= 2, 512 of 1 at M = 3-4
    {2560, 4096, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 2, 4, 5, 1)},
    {2560, 4096, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 8, 5, 1)},
    {2560, 4096, KRK_EPILOGUE_NONE, 3, 4, kcfg(KRK_KERNEL_VALU, 1, 4, 5, 1)},
    // M = 5-32: the wave-sliced kernel on 256 blocks of 10 channels, K
    // unsplit, 128-k chunks up to M = 12 and 64-k chunks above, 2 in flight
    // per wave (M = 8: 6.6 against 7.3 us on the VALU kernel; M = 20: 8.2
    // against 9.2 us with x held in registers on 160 LDS-staged blocks);
    // above, 3 stages in flight up to three x tiles, 2 with four (1-5%
    // faster each way)
    {2560, 4096, KRK_EPILOGUE_NONE, 5, 12, kcfg(KRK_KERNEL_SLICE, 0, 2, 0, 1, 128, 10)},
    {2560, 4096, KRK_EPILOGUE_NONE, 13, 32, kcfg(KRK_KERNEL_SLICE, 0, 2, 0, 1, 64, 10)},
    {2560, 4096, KRK_EPILOGUE_NONE, 33, 48, kcfg(KRK_KERNEL_MFMA_LDS, 2, 3, 0, 3, 256)},
    {2560, 4096, KRK_EPILOGUE_NONE, 49, 64, kcfg(KRK_KERNEL_MFMA_LDS, 2, 2, 0, 3, 256)},
    // gate_up 2560 -> 2 x 9728 with SiLU*mul
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 1, 1, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 0, 2, 1)},
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 3, 4, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    // M = 5-16: the stream kernel, 5 ring slots (M = 5-8 18.7-19.1 us against
    // 20.0-22.9 us for the VALU plan in three alternating passes, once the
    // stream kernel's block epilogue batched its reads).  M = 17-32 (two x
    // tiles): 4 ring slots, 0.2-0.3 us under 5 at M = 20, 24, 28 and 32 in
    // three alternating passes once the stream kernel's multi-tile stages
    // lost their workgroup barrier; 5 elsewhere.
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 5, 16, kcfg(KRK_KERNEL_STREAM, 1, 5, 0, 1)},
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 17, 32, kcfg(KRK_KERNEL_STREAM, 1, 4, 0, 1)},
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 33, 64, kcfg(KRK_KERNEL_STREAM, 1, 5, 0, 1)},
    // down 9728 -> 2560
    {2560, 9728, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 1, 0, 5, 1)},
    // M = 2-12: the wave-sliced kernel on 256 blocks of 10 channels, K
    // unsplit, 128-k chunks, 2 in flight per wave (M = 2: 9.9 against 11.1 us
    // on the VALU kernel; M = 8: 10.8 against 12.9 us); M = 13-24: 128
    // blocks of 20 channels in 2 K splits, 64-k chunks (2-3% under the
    // LDS-staged plans)
    {2560, 9728, KRK_EPILOGUE_NONE, 2, 12, kcfg(KRK_KERNEL_SLICE, 0, 2, 0, 1, 128, 10)},
    {2560, 9728, KRK_EPILOGUE_NONE, 13, 24, kcfg(KRK_KERNEL_SLICE, 0, 2, 0, 2, 64, 20)},
    {2560, 9728, KRK_EPILOGUE_NONE, 25, 48, kcfg(KRK_KERNEL_MFMA_LDS, 2, 3, 0, 3, 256)},
    {2560, 9728, KRK_EPILOGUE_NONE, 49, 64, kcfg(KRK_KERNEL_MFMA_LDS, 2, 2, 0, 3, 256)},
    // lm_head 2560 -> 151936
    {151936, 2560, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 1, 0, 8, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 4, 0, 4, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 3, 4, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    // 7 stages in the ring with one x tile (4-5% faster than 5), 5 with two
    {151936, 2560, KRK_EPILOGUE_NONE, 5, 16, kcfg(KRK_KERNEL_STREAM, 1, 7, 0, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 17, 32, kcfg(KRK_KERNEL_STREAM, 1, 5, 0, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 33, 64, kcfg(KRK_KERNEL_STREAM, 1, 5, 0, 1)},

    // One GPU's shard under 8-way tensor parallelism (QKV, gate_up and
    // lm_head split along N, o and down along K), from the warm-up tuner's
    // full search on an MI355X (graph replay over >= 300 MB of weight copies).
    // qkv shard 2560 -> 768 (M = 9-32: x held in registers, 8-17% faster)
    {768, 2560, KRK_EPILOGUE_NONE, 1, 8, kcfg(KRK_KERNEL_VALU, 1, 0, 4, 1)},
    {768, 2560, KRK_EPILOGUE_NONE, 9, 32, kcfg(KRK_KERNEL_MFMA_LDS, 1, 3, 0, 1, 512, 16, 2)},
    {768, 2560, KRK_EPILOGUE_NONE, 33, 64, kcfg(KRK_KERNEL_MFMA_LDS, 1, 2, 0, 4, 256)},
    // o shard 512 -> 2560
    {2560, 512, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 2, 0, 4, 1)},
    {2560, 512, KRK_EPILOGUE_NONE, 2, 4, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    {2560, 512, KRK_EPILOGUE_NONE, 5, 16, kcfg(KRK_KERNEL_MFMA, 1, 4, 4, 1)},
    {2560, 512, KRK_EPILOGUE_NONE, 17, 48, kcfg(KRK_KERNEL_MFMA_LDS, 1, 2, 0, 1, 512)},
    {2560, 512, KRK_EPILOGUE_NONE, 49, 64, kcfg(KRK_KERNEL_MFMA_LDS, 1, 2, 0, 1, 256)},
    // gate_up shard 2560 -> 2 x 1216 with SiLU*mul
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 1, 2, kcfg(KRK_KERNEL_VALU, 2, 0, 5, 1)},
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 3, 4, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 5, 8, kcfg(KRK_KERNEL_VALU, 4, 0, 4, 1)},
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 9, 16, kcfg(KRK_KERNEL_STREAM, 1, 5, 0, 1)},
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 17, 32, kcfg(KRK_KERNEL_MFMA_LDS, 2, 2, 0, 1, 512, 8)},
    {2432, 2560, KRK_EPILOGUE_SILU_MUL, 33, 64, kcfg(KRK_KERNEL_MFMA_LDS, 2, 2, 0, 3, 256)},
    // down shard 1216 -> 2560
    {2560, 1216, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 4, 0, 4, 1)},
    {2560, 1216, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 0, 4, 1)},
    {2560, 1216, KRK_EPILOGUE_NONE, 3, 4, kcfg(KRK_KERNEL_VALU, 1, 0, 4, 1)},
    {2560, 1216, KRK_EPILOGUE_NONE, 5, 48, kcfg(KRK_KERNEL_MFMA_LDS, 1, 3, 0, 1, 256)},
    {2560, 1216, KRK_EPILOGUE_NONE, 49, 64, kcfg(KRK_KERNEL_MFMA_LDS, 1, 2, 0, 1, 256)},
    // lm_head shard 2560 -> 18992
    {18992, 2560, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 1, 0, 4, 1)},
    {18992, 2560, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 0, 8, 1)},
    {18992, 2560, KRK_EPILOGUE_NONE, 3, 8, kcfg(KRK_KERNEL_VALU, 4, 0, 4, 1)},
    {18992, 2560, KRK_EPILOGUE_NONE, 9, 24, kcfg(KRK_KERNEL_STREAM, 1, 4, 0, 1)},
    {18992, 2560, KRK_EPILOGUE_NONE, 25, 48, kcfg(KRK_KERNEL_STREAM, 1, 4, 0, 1)},
    {18992, 2560, KRK_EPILOGUE_NONE, 49, 64, kcfg(KRK_KERNEL_STREAM, 1, 3, 0, 1)},
};

// VALU: x rows held per launch (a power of two >= M), and the instantiated
// numbers of 512-element blocks in flight per W row.
inline int valu_mx(int Mc) { return Mc <= 1 ? 1 : Mc <= 2 ? 2 : Mc <= 4 ? 4 : 8; }
constexpr int kValuDepths[] = {2, 3, 4, 5, 7, 8, 10, 19};
// Loads a lane keeps in flight: D blocks of R W rows, plus MX x rows when x
// stays in registers (MX < 4).  48 keeps the kernels within 256 VGPRs.
inline int valu_loads(int MX, int R, int D) { return (MX < krk::kValuLdsMinRows ? MX + R : R) * D; }
inline bool valu_depth_ok(int MX, int R, int D) {
    for (int d : kValuDepths)
        if (d == D) return valu_loads(MX, R, D) <= 48;
    return false;
}
// Smallest depth covering a split's blocks in one pass, else the deepest.
inline int valu_depth(int MX, int R, int blocks) {
    int best = 0;
    for (int d : kValuDepths) {
        if (valu_loads(MX, R, d) > 48) break;
        best = d;
        if (d >= blocks) break;
    }
    return best;
}

int stream_xs(int MT, int nst);

// MFMA_LDS k per stage when the caller or the table does not choose one.
inline int default_kc(int MT, int NT) { return krk::mfma_lds_kc_ok(MT, NT, 512) ? 512 : 256; }

void auto_config(int M, int N, int K, int epilogue, krk_gemm_config* c) {
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    const bool silu = epilogue == KRK_EPILOGUE_SILU_MUL;
    const int mt = cdiv(Mc, 16);
    const int KST = cdiv(K, 512);
    for (const TableEntry& e : kTable) {
        if (e.N == N && e.K == K && e.epilogue == epilogue && Mc >= e.m_lo && Mc <= e.m_hi) {
            *c = e.cfg;
            c->m_tiles = mt;
            if (c->kernel == KRK_KERNEL_MFMA_LDS) {
                c->waves = krk::kLdsWaves;
                c->unroll = c->unroll ? c->unroll : 2;
                c->k_chunk = c->k_chunk ? c->k_chunk : default_kc(mt, c->n_tiles);
                c->channels = c->channels ? c->channels : 16 * (silu ? c->n_tiles / 2 : c->n_tiles);
                c->x_preload = c->x_preload ? c->x_preload : 1;
            }
            if (c->kernel == KRK_KERNEL_STREAM) c->waves = 8;
            if (c->kernel == KRK_KERNEL_SLICE) {
                const SliceShape v = slice_shape(c->k_chunk, c->channels, Mc);
                c->waves = krk::kSliceWaves;
                c->n_tiles = v.NT;
                c->m_tiles = v.MT;
            }
            if (c->kernel == KRK_KERNEL_VALU) {
                c->m_tiles = valu_mx(Mc);
                if (!c->unroll) c->unroll = valu_depth(c->m_tiles, c->n_tiles, cdiv(KST, c->splits));
            }
            return;
        }
    }
    // Other shapes.  M <= 8: the VALU row-streaming kernel, K split until
    // about 600 workgroup-splits stream and the x slice fits LDS.  Larger M:
    // the persistent stream kernel where x is large and the weight stream
    // long (its x-in-registers design pays off), otherwise the LDS-staged
    // MFMA kernel with K split until ~200 workgroups stream.
    const int Nout = silu ? N / 2 : N;
    krk_gemm_config r{};
    r.m_tiles = mt;
    if (Mc <= kValuMaxRows) {
        r.kernel = KRK_KERNEL_VALU;
        r.m_tiles = valu_mx(Mc);
        r.n_tiles = (silu || Mc > 4) ? 2 : 1;
        r.waves = 4;
        const int nblocks = cdiv(Nout, r.waves * (silu ? r.n_tiles / 2 : r.n_tiles));
        r.splits = 1;
        while (r.splits < KST && r.splits < 32 &&
               (nblocks * r.splits < 600 || krk::valu_lds_bytes(r.m_tiles, cdiv(KST, r.splits)) > kLdsBudget))
            ++r.splits;
        r.unroll = valu_depth(r.m_tiles, r.n_tiles, cdiv(KST, r.splits));
    } else if (Mc > 32 && (silu || N >= 65536)) {
        r.kernel = KRK_KERNEL_STREAM;
        r.n_tiles = 1;
        r.waves = 8;
        r.unroll = 4;
        r.splits = 1;
        while (r.splits < 32 && stream_xs(mt, cdiv(KST, r.splits)) == 0) ++r.splits;
    } else {
        r.kernel = KRK_KERNEL_MFMA_LDS;
        r.n_tiles = (N >= 65536 && Mc > 8) ? 4 : 2;
        r.unroll = 2;
        r.k_chunk = default_kc(mt, r.n_tiles);
        r.waves = krk::kLdsWaves;
        r.channels = 16 * (silu ? r.n_tiles / 2 : r.n_tiles);
        r.x_preload = 1;
        const int nblocks = cdiv(Nout, r.channels);
        r.splits = 1;
        while (nblocks * r.splits < 192 && r.splits < 4 && KST >= 2 * (r.splits + 1)) ++r.splits;
    }
    *c = r;
}

// MFMA_LDS keeps `unroll` stages of row pieces in registers; three stages fit
// 256 VGPRs without spilling up to this many 16-row tiles (m + n).
constexpr int kLdsPf3MaxTiles = 6;
constexpr bool mfma_lds_pf3(int MT, int NT) { return MT + NT <= kLdsPf3MaxTiles; }
// MFMA_LDS with x held in registers for the whole K (x_preload = 2): 512-k
// stages, K unsplit in at most kLdsXpreStages of them, up to two x tiles.
constexpr int kLdsXpreMaxMTiles = 2;
inline bool lds_xpre_ok(const krk_gemm_config& c, int K) {
    const int most = c.m_tiles == 1 && c.n_tiles == 1 ? krk::kLdsXpreLongStages : krk::kLdsXpreStages;
    return c.k_chunk == 512 && c.splits == 1 && cdiv(K, 512) <= most && c.m_tiles <= kLdsXpreMaxMTiles;
}

// Dynamic LDS a gfx950 workgroup may use: 160 KB less room for the kernels'
// static __shared__ variables.
constexpr size_t kLdsMax = 163840 - kLdsReserve;

// STREAM: x fragments live in 8·XS·MT VGPRs per lane; the instantiated XS
// values per MT are the ones that stay within 256 VGPRs without spilling in
// the stage loop (MT=4, XS=5 spills a few bytes outside it).
int stream_xs(int MT, int nst) {
    static const int kXs[4][4] = {{4, 5, 8, 10}, {4, 5, 8, 0}, {4, 5, 0, 0}, {4, 5, 0, 0}};
    for (int xs : kXs[MT - 1])
        if (xs && xs >= nst) return xs;
    return 0;
}
// Deepest ring that leaves room for one output-buffer block.
inline int stream_max_depth(int MT, int nred) {
    int d = krk::kStreamMaxDepth;
    while (d > 2 && krk::stream_lds_bytes(MT, d, nred) + krk::stream_out_bytes(MT, false) > kLdsMax) --d;
    return d;
}
// Reduction areas of a stream launch: one when every split owns two or more
// K stages.
inline int stream_nred_for(int K, int splits) { return krk::stream_nred(cdiv(K, krk::kStreamKC) / splits); }
// Persistent grid: workgroups per split, at most one per CU, chosen so the
// blocks divide as evenly as possible (a 1.25x overload costs more than
// leaving CUs idle).
inline int stream_groups(int nblocks, int splits) {
    const int cap = kCuCount / splits > 0 ? kCuCount / splits : 1;
    if (nblocks <= cap) return nblocks;
    int best = cap;
    double best_eff = 0.0;
    for (int g = cap; g >= cap / 2 && g >= 1; --g) {
        const int per = cdiv(nblocks, g);
        const double eff = (double)nblocks / ((double)per * kCuCount / splits);
        if (eff > best_eff + 1e-9) { best_eff = eff; best = g; }
    }
    return best;
}

// Fill the zero fields of a caller's configuration from the table and check
// that the result is one this build instantiates.
int resolve_config(int M, int N, int K, int epilogue, const krk_gemm_config* in, krk_gemm_config* out) {
    krk_gemm_config a;
    auto_config(M, N, K, epilogue, &a);
    if (!in) { *out = a; return KRK_OK; }
    krk_gemm_config c = *in;
    if (c.prologue != 0 && c.prologue != 1)
        return fail(KRK_ERR_UNSUPPORTED, "prologue=%d not in {0, 1}", c.prologue);
    if (c.kernel == KRK_KERNEL_AUTO) c.kernel = a.kernel;
    if (c.kernel != KRK_KERNEL_MFMA_LDS) c.x_preload = 0;  // MFMA_LDS only
    const bool same_kernel = c.kernel == a.kernel;
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    if (c.kernel == KRK_KERNEL_MFMA) {
        if (!c.m_tiles) c.m_tiles = cdiv(Mc, 16);
        if (!c.n_tiles) c.n_tiles = same_kernel ? a.n_tiles : (epilogue == KRK_EPILOGUE_SILU_MUL ? 2 : 1);
        if (!c.unroll) c.unroll = same_kernel ? a.unroll : 4;
        if (!c.waves) c.waves = same_kernel ? a.waves : 4;
        if (!c.splits) c.splits = same_kernel ? a.splits : 1;
        if (c.m_tiles < cdiv(Mc, 16) || c.m_tiles > 4)
            return fail(KRK_ERR_INVALID, "m_tiles=%d cannot cover %d rows (need %d..4)", c.m_tiles, Mc, cdiv(Mc, 16));
        if (c.n_tiles != 1 && c.n_tiles != 2 && c.n_tiles != 4)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA n_tiles=%d not in {1,2,4}", c.n_tiles);
        if (epilogue == KRK_EPILOGUE_SILU_MUL && c.n_tiles % 2)
            return fail(KRK_ERR_UNSUPPORTED, "SILU_MUL needs an even n_tiles, got %d", c.n_tiles);
        if (c.unroll != 2 && c.unroll != 4 && c.unroll != 8)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA unroll=%d not in {2,4,8}", c.unroll);
        if (c.waves > 0 && (size_t)c.waves * c.m_tiles * c.n_tiles * 1024 + kLdsReserve > kLdsBudget)
            return fail(KRK_ERR_UNSUPPORTED, "waves*m_tiles*n_tiles=%d KB of reduction LDS exceeds the %zu-byte budget",
                        c.waves * c.m_tiles * c.n_tiles, kLdsBudget);
    } else if (c.kernel == KRK_KERNEL_MFMA_LDS) {
        if (!c.m_tiles) c.m_tiles = cdiv(Mc, 16);
        if (!c.n_tiles) c.n_tiles = same_kernel ? a.n_tiles : (epilogue == KRK_EPILOGUE_SILU_MUL ? 2 : 1);
        if (!c.unroll) c.unroll = same_kernel ? a.unroll : 2;
        if (!c.waves) c.waves = krk::kLdsWaves;
        if (!c.k_chunk) c.k_chunk = same_kernel && a.m_tiles == c.m_tiles && a.n_tiles == c.n_tiles ? a.k_chunk
                                                                                                  : default_kc(c.m_tiles, c.n_tiles);
        if (!c.splits) c.splits = same_kernel ? a.splits : 1;
        if (c.m_tiles < cdiv(Mc, 16) || c.m_tiles > 4)
            return fail(KRK_ERR_INVALID, "m_tiles=%d cannot cover %d rows (need %d..4)", c.m_tiles, Mc, cdiv(Mc, 16));
        if (c.n_tiles != 1 && c.n_tiles != 2 && c.n_tiles != 4)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS n_tiles=%d not in {1,2,4}", c.n_tiles);
        if (epilogue == KRK_EPILOGUE_SILU_MUL && c.n_tiles % 2)
            return fail(KRK_ERR_UNSUPPORTED, "SILU_MUL needs an even n_tiles, got %d", c.n_tiles);
        if (c.waves != krk::kLdsWaves)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS runs %d waves per workgroup, got waves=%d", krk::kLdsWaves, c.waves);
        if (!krk::mfma_lds_kc_ok(c.m_tiles, c.n_tiles, c.k_chunk))
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS k_chunk=%d: 256, or 512 when m_tiles + n_tiles <= 4 (%d + %d)",
                        c.k_chunk, c.m_tiles, c.n_tiles);
        if (c.unroll != 2 && !(c.unroll == 3 && mfma_lds_pf3(c.m_tiles, c.n_tiles)))
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS stages in flight (unroll)=%d not instantiated for %d x %d tiles "
                        "(2, or 3 when m_tiles + n_tiles <= %d)", c.unroll, c.m_tiles, c.n_tiles, kLdsPf3MaxTiles);
        if (c.splits < 1 || c.splits > 32)
            return fail(KRK_ERR_UNSUPPORTED, "splits=%d not in 1..32", c.splits);
        const int full = 16 * (epilogue == KRK_EPILOGUE_SILU_MUL ? c.n_tiles / 2 : c.n_tiles);
        if (!c.channels) c.channels = same_kernel && a.n_tiles == c.n_tiles && a.channels ? a.channels : full;
        if (c.channels < 8 || c.channels > full || c.channels % 8)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS channels=%d: a multiple of 8 in 8..%d for %d tiles", c.channels,
                        full, c.n_tiles);
        if (!c.x_preload) c.x_preload = same_kernel && a.x_preload == 2 && lds_xpre_ok(c, K) ? 2 : 1;
        if (c.x_preload != 1 && c.x_preload != 2)
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS x_preload=%d not in {1, 2}", c.x_preload);
        if (c.x_preload == 2 && !lds_xpre_ok(c, K))
            return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS x_preload=2 needs k_chunk 512, splits 1, K <= %d and m_tiles <= %d",
                        krk::kLdsXpreStages * 512, kLdsXpreMaxMTiles);
        *out = c;
        return KRK_OK;
    } else if (c.kernel == KRK_KERNEL_STREAM) {
        if (!c.m_tiles) c.m_tiles = cdiv(Mc, 16);
        c.n_tiles = 1;
        c.waves = krk::kStreamWaves;
        if (!c.splits) c.splits = same_kernel ? a.splits : 1;
        if (c.m_tiles < cdiv(Mc, 16) || c.m_tiles > 4)
            return fail(KRK_ERR_INVALID, "m_tiles=%d cannot cover %d rows (need %d..4)", c.m_tiles, Mc, cdiv(Mc, 16));
        if (c.splits < 1 || c.splits > 32)
            return fail(KRK_ERR_UNSUPPORTED, "splits=%d not in 1..32", c.splits);
        // Every split must own at least one K stage: a workgroup of an empty
        // split would not take part in its blocks' fix-up.
        if (c.splits > cdiv(K, krk::kStreamKC))
            return fail(KRK_ERR_UNSUPPORTED, "STREAM splits=%d exceeds the %d K stages of %d elements", c.splits,
                        cdiv(K, krk::kStreamKC), krk::kStreamKC);
        if (stream_xs(c.m_tiles, cdiv(cdiv(K, krk::kStreamKC), c.splits)) == 0)
            return fail(KRK_ERR_UNSUPPORTED, "STREAM keeps x in registers: %d K stages per split x %d m tiles is too "
                        "many (raise splits)", cdiv(cdiv(K, krk::kStreamKC), c.splits), c.m_tiles);
        const int maxd = stream_max_depth(c.m_tiles, stream_nred_for(K, c.splits));
        if (!c.unroll) c.unroll = same_kernel && a.unroll ? a.unroll : maxd;
        if (c.unroll < 2 || c.unroll > maxd)
            return fail(KRK_ERR_UNSUPPORTED, "STREAM depth (unroll) %d not in 2..%d", c.unroll, maxd);
        *out = c;
        return KRK_OK;
    } else if (c.kernel == KRK_KERNEL_SLICE) {
        if (epilogue != KRK_EPILOGUE_NONE)
            return fail(KRK_ERR_UNSUPPORTED, "SLICE computes plain projections (no SILU_MUL epilogue)");
        if (Mc > kSliceMaxRows)
            return fail(KRK_ERR_UNSUPPORTED, "SLICE handles M <= %d per launch, got %d", kSliceMaxRows, Mc);
        if (!c.k_chunk) c.k_chunk = same_kernel ? a.k_chunk : 64;
        if (c.k_chunk != 64 && c.k_chunk != 128)
            return fail(KRK_ERR_UNSUPPORTED, "SLICE k_chunk=%d not in {64, 128}", c.k_chunk);
        if (!c.channels) {
            const int per_cu = cdiv(N, kCuCount);
            c.channels = same_kernel ? a.channels : (per_cu < kSliceMaxChannels ? per_cu : kSliceMaxChannels);
        }
        if (c.channels < 1 || c.channels > kSliceMaxChannels)
            return fail(KRK_ERR_UNSUPPORTED, "SLICE channels=%d not in 1..%d", c.channels, kSliceMaxChannels);
        if (!c.unroll) c.unroll = same_kernel ? a.unroll : 2;
        if (!c.splits) c.splits = same_kernel ? a.splits : 1;
        c.waves = krk::kSliceWaves;
        const SliceShape v = slice_shape(c.k_chunk, c.channels, Mc);
        c.n_tiles = v.NT;
        c.m_tiles = v.MT;
        const int nch = cdiv(K, c.k_chunk);
        if (c.splits < 1 || c.splits > 32 || c.splits > nch)
            return fail(KRK_ERR_UNSUPPORTED, "SLICE splits=%d not in 1..min(32, %d chunks of %d k)", c.splits, nch,
                        c.k_chunk);
        if (!slice_inst(c.k_chunk, v.NT, v.NGV, v.XGV, c.unroll))
            return fail(KRK_ERR_UNSUPPORTED, "SLICE variant not instantiated: k_chunk=%d, %d channels, %d rows, %d "
                        "chunks in flight (64-k chunks: up to 32 channels and rows, 2 or 3 in flight within 160 KB "
                        "of LDS; 128-k chunks: up to 16 of each, 2 in flight)", c.k_chunk, c.channels, Mc, c.unroll);
        *out = c;
        return KRK_OK;
    } else if (c.kernel == KRK_KERNEL_VALU) {
        if (Mc > kValuMaxRows)
            return fail(KRK_ERR_UNSUPPORTED, "VALU kernel handles M <= %d, got %d", kValuMaxRows, M);
        const bool silu = epilogue == KRK_EPILOGUE_SILU_MUL;
        c.m_tiles = valu_mx(Mc);
        if (!c.n_tiles) c.n_tiles = same_kernel ? a.n_tiles : 2;
        if (!c.waves) c.waves = same_kernel ? a.waves : 8;
        if (!c.splits) c.splits = same_kernel ? a.splits : 1;
        if (c.n_tiles != 1 && c.n_tiles != 2 && c.n_tiles != 4)
            return fail(KRK_ERR_UNSUPPORTED, "VALU n_tiles (W rows per wave)=%d not in {1,2,4}", c.n_tiles);
        if (silu && c.n_tiles % 2)
            return fail(KRK_ERR_UNSUPPORTED, "SILU_MUL needs an even n_tiles (gate and up rows), got %d", c.n_tiles);
        if (c.waves < 1 || c.waves > krk::kValuMaxWaves)
            return fail(KRK_ERR_UNSUPPORTED, "VALU waves=%d not in 1..%d", c.waves, krk::kValuMaxWaves);
        const int nb = cdiv(K, krk::kValuBlock);
        if (c.splits < 1 || c.splits > 32 || c.splits > nb)
            return fail(KRK_ERR_UNSUPPORTED, "VALU splits=%d not in 1..min(32, %d K blocks)", c.splits, nb);
        const int per = cdiv(nb, c.splits);
        if (!c.unroll) c.unroll = valu_depth(c.m_tiles, c.n_tiles, per);
        if (!valu_depth_ok(c.m_tiles, c.n_tiles, c.unroll))
            return fail(KRK_ERR_UNSUPPORTED, "VALU unroll (blocks in flight)=%d not instantiated for %d rows per wave",
                        c.unroll, c.n_tiles);
        if (krk::valu_lds_bytes(c.m_tiles, per) > kLdsMax)
            return fail(KRK_ERR_UNSUPPORTED, "VALU x slice of %zu bytes exceeds LDS (raise splits)",
                        krk::valu_lds_bytes(c.m_tiles, per));
        *out = c;
        return KRK_OK;
    } else {
        return fail(KRK_ERR_UNSUPPORTED, "unknown kernel %d", c.kernel);
    }
    if (c.waves != 1 && c.waves != 2 && c.waves != 4)
        return fail(KRK_ERR_UNSUPPORTED, "waves=%d not in {1,2,4}", c.waves);
    if (c.splits < 1 || c.splits > 32)
        return fail(KRK_ERR_UNSUPPORTED, "splits=%d not in 1..32", c.splits);
    *out = c;
    return KRK_OK;
}

// Workspace layout: [block counters, padded to 256 B][fp32 partials splits x Mc x N].
size_t workspace_for(int M, int N, int epilogue, const krk_gemm_config& c) {
    if (c.splits <= 1) return 0;
    const Geometry g = geometry(M, N, epilogue, c);
    return align_up((size_t)g.nblocks * sizeof(uint32_t), 256) +
           (size_t)c.splits * (size_t)g.Mc * (size_t)N * sizeof(float);
}

bool overlaps(uintptr_t a0, uintptr_t a1, uintptr_t b0, uintptr_t b1) { return a0 < b1 && b0 < a1; }

struct LaunchArgs {
    const uint16_t* x;
    int64_t ldx;
    const uint16_t* w;
    int64_t ldw;
    uint16_t* y;
    int64_t ldy;
    int M, N, K, splits;
    int cb;  // output channels per block (MFMA_LDS)
    float* part;
    uint32_t* ctr;
};

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return KRK_OK;
    return fail(KRK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Raise a kernel's dynamic-LDS limit to `bytes` on the calling thread's
// current device, once per device and kernel (the attribute is set in the
// device's context, so a process that drives several GPUs needs it on each).
// `done` is the kernel's own set of devices already configured.
hipError_t ensure_lds_limit(const void* fn, int bytes, std::atomic<uint64_t>& done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
    return e;
}

template <int MT, int NT, int U, bool SILU>
int launch_mfma(const LaunchArgs& a, int nblocks, int waves, hipStream_t stream) {
    void* args[] = {(void*)&a.x, (void*)&a.ldx, (void*)&a.w,      (void*)&a.ldw, (void*)&a.y,    (void*)&a.ldy,
                    (void*)&a.M, (void*)&a.N,   (void*)&a.K,      (void*)&a.splits, (void*)&a.part, (void*)&a.ctr};
    const size_t shm = (size_t)waves * MT * NT * 64 * sizeof(krk::f32x4);
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&krk::mfma_gemm_kernel<MT, NT, U, SILU>),
                                   dim3(nblocks * a.splits), dim3(64 * waves), args, shm, stream);
    return hip_status(e, "mfma_gemm_kernel launch");
}

template <int MT, int NT, bool SILU>
int dispatch_mfma_u(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    switch (c.unroll) {
        case 2: return launch_mfma<MT, NT, 2, SILU>(a, nblocks, c.waves, s);
        case 4: return launch_mfma<MT, NT, 4, SILU>(a, nblocks, c.waves, s);
        case 8: return launch_mfma<MT, NT, 8, SILU>(a, nblocks, c.waves, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "MFMA unroll=%d", c.unroll);
}

template <int MT, bool SILU>
int dispatch_mfma_n(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if constexpr (!SILU) {
        if (c.n_tiles == 1) return dispatch_mfma_u<MT, 1, false>(a, c, nblocks, s);
    }
    if (c.n_tiles == 2) return dispatch_mfma_u<MT, 2, SILU>(a, c, nblocks, s);
    if (c.n_tiles == 4) return dispatch_mfma_u<MT, 4, SILU>(a, c, nblocks, s);
    return fail(KRK_ERR_UNSUPPORTED, "MFMA n_tiles=%d", c.n_tiles);
}

template <bool SILU>
int dispatch_mfma(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    switch (c.m_tiles) {
        case 1: return dispatch_mfma_n<1, SILU>(a, c, nblocks, s);
        case 2: return dispatch_mfma_n<2, SILU>(a, c, nblocks, s);
        case 3: return dispatch_mfma_n<3, SILU>(a, c, nblocks, s);
        case 4: return dispatch_mfma_n<4, SILU>(a, c, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "MFMA m_tiles=%d", c.m_tiles);
}

template <int MT, int NT, int PF, int KC, bool SILU, bool SEL = false, bool NORM = false, int XPRE = 0>
int launch_mfma_lds(const LaunchArgs& a, int nblocks, hipStream_t stream, krk::SelectArgs sa = {},
                    krk::NormArgs na = {}) {
    if constexpr ((PF == 3 && !mfma_lds_pf3(MT, NT)) || !krk::mfma_lds_kc_ok(MT, NT, KC)) {
        return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS unroll=%d k_chunk=%d with %d x %d tiles", PF, KC, MT, NT);
    } else {
        const void* fn = reinterpret_cast<const void*>(&krk::mfma_lds_kernel<MT, NT, PF, KC, SILU, SEL, NORM, XPRE>);
        const size_t shm = krk::mfma_lds_bytes(MT, NT, KC, SEL);
        // Tiles above 64 KB use gfx950's larger LDS; the limit is raised once
        // per instantiation (a function attribute, not a stream operation).
        static std::atomic<uint64_t> done{0};
        const hipError_t attr = shm > 65536 ? ensure_lds_limit(fn, (int)shm, done) : hipSuccess;
        if (attr != hipSuccess) return hip_status(attr, "mfma_lds_kernel LDS attribute");
        int cb = a.cb;
        void* args[] = {(void*)&a.x, (void*)&a.ldx, (void*)&a.w,      (void*)&a.ldw, (void*)&a.y,    (void*)&a.ldy,
                        (void*)&a.M, (void*)&a.N,   (void*)&a.K,      (void*)&a.splits, (void*)&cb, (void*)&a.part,
                        (void*)&a.ctr, (void*)&sa, (void*)&na};
        hipError_t e = hipLaunchKernel(fn, dim3(nblocks * a.splits), dim3(64 * krk::kLdsWaves), args, shm, stream);
        return hip_status(e, "mfma_lds_kernel launch");
    }
}

template <int MT, int NT, int KC, bool SILU>
int dispatch_mfma_lds_pf(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if (c.unroll == 3) return launch_mfma_lds<MT, NT, 3, KC, SILU>(a, nblocks, s);
    return launch_mfma_lds<MT, NT, 2, KC, SILU>(a, nblocks, s);
}

// x held in registers for the whole K (x_preload = 2; 512-k stages).
template <int MT, int NT, bool SILU>
int dispatch_mfma_lds_xpre(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if constexpr (MT <= kLdsXpreMaxMTiles && krk::mfma_lds_kc_ok(MT, NT, 512)) {
        // The loop runs all of the held stages: 5 where K fits them, else 8.
        if (cdiv(a.K, 512) <= krk::kLdsNormStages) {
            if (c.unroll == 3) return launch_mfma_lds<MT, NT, 3, 512, SILU, false, false, krk::kLdsNormStages>(a, nblocks, s);
            return launch_mfma_lds<MT, NT, 2, 512, SILU, false, false, krk::kLdsNormStages>(a, nblocks, s);
        }
        if (cdiv(a.K, 512) <= krk::kLdsXpreStages) {
            if (c.unroll == 3) return launch_mfma_lds<MT, NT, 3, 512, SILU, false, false, krk::kLdsXpreStages>(a, nblocks, s);
            return launch_mfma_lds<MT, NT, 2, 512, SILU, false, false, krk::kLdsXpreStages>(a, nblocks, s);
        }
        if constexpr (MT == 1 && NT == 1) {
            constexpr int XL = krk::kLdsXpreLongStages;
            if (c.unroll == 3) return launch_mfma_lds<MT, NT, 3, 512, SILU, false, false, XL>(a, nblocks, s);
            return launch_mfma_lds<MT, NT, 2, 512, SILU, false, false, XL>(a, nblocks, s);
        }
        return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS x_preload=2 with %d x tiles and %d stages", MT, cdiv(a.K, 512));
    } else {
        return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS x_preload=2 with %d x %d tiles", MT, NT);
    }
}

template <int MT, int NT, bool SILU>
int dispatch_mfma_lds_kc(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if (c.k_chunk == 512) {
        if (c.x_preload == 2) return dispatch_mfma_lds_xpre<MT, NT, SILU>(a, c, nblocks, s);
        return dispatch_mfma_lds_pf<MT, NT, 512, SILU>(a, c, nblocks, s);
    }
    return dispatch_mfma_lds_pf<MT, NT, 256, SILU>(a, c, nblocks, s);
}

template <int MT, bool SILU>
int dispatch_mfma_lds_n(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if constexpr (!SILU) {
        if (c.n_tiles == 1) return dispatch_mfma_lds_kc<MT, 1, false>(a, c, nblocks, s);
    }
    if (c.n_tiles == 2) return dispatch_mfma_lds_kc<MT, 2, SILU>(a, c, nblocks, s);
    if (c.n_tiles == 4) return dispatch_mfma_lds_kc<MT, 4, SILU>(a, c, nblocks, s);
    return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS n_tiles=%d", c.n_tiles);
}

template <bool SILU>
int dispatch_mfma_lds(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    switch (c.m_tiles) {
        case 1: return dispatch_mfma_lds_n<1, SILU>(a, c, nblocks, s);
        case 2: return dispatch_mfma_lds_n<2, SILU>(a, c, nblocks, s);
        case 3: return dispatch_mfma_lds_n<3, SILU>(a, c, nblocks, s);
        case 4: return dispatch_mfma_lds_n<4, SILU>(a, c, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS m_tiles=%d", c.m_tiles);
}

template <int MT, int XS, bool SILU, int SK = 0, bool XF = false>
int launch_stream(const LaunchArgs& a, int nblocks, int depth, hipStream_t stream, krk::SelectArgs sa = {}) {
    const void* fn = reinterpret_cast<const void*>(&krk::stream_gemm_kernel<MT, XS, SILU, SK, XF>);
    int nred = stream_nred_for(a.K, a.splits);
    const int G = stream_groups(nblocks, a.splits);
    // Two or more x tiles: a second reduction area when it fits beside the
    // ring and every output block (the kernel then needs no barrier at a
    // block's second stage).
    if (MT >= 2 && nred == 1) {
        const size_t out = a.splits == 1 ? (size_t)cdiv(nblocks, G) * krk::stream_out_bytes(MT, SILU) : 0;
        if (krk::stream_lds_bytes(MT, depth, 2) + out <= kLdsMax) nred = 2;
    }
    size_t shm = krk::stream_lds_bytes(MT, depth, nred);
    // Unsplit K: the rest of the LDS holds finished blocks until the end.
    int obcap = 0;
    if (a.splits == 1) {
        const size_t per = krk::stream_out_bytes(MT, SILU);
        const size_t room = shm < kLdsMax ? (kLdsMax - shm) / per : 0;
        const int blocks_per_wg = cdiv(nblocks, G);
        obcap = (int)(room < (size_t)blocks_per_wg ? room : (size_t)blocks_per_wg);
        shm += (size_t)obcap * per;
    }
    if (shm > kLdsMax || (a.splits == 1 && obcap < 1))
        return fail(KRK_ERR_UNSUPPORTED, "STREAM depth %d leaves no LDS for the output buffer", depth);
    // The x preload stages its rows from the start of the area, before the ring.
    if (!XF && shm < krk::stream_xstage_bytes(MT, XS)) shm = krk::stream_xstage_bytes(MT, XS);
    static std::atomic<uint64_t> done{0};
    const hipError_t attr = ensure_lds_limit(fn, (int)kLdsMax, done);
    if (attr != hipSuccess) return hip_status(attr, "stream_gemm_kernel LDS attribute");
    const int groups = G * a.splits;
    void* args[] = {(void*)&a.x, (void*)&a.ldx, (void*)&a.w, (void*)&a.ldw, (void*)&a.y, (void*)&a.ldy,
                    (void*)&a.M, (void*)&a.N,   (void*)&a.K, (void*)&a.splits, (void*)&depth, (void*)&obcap,
                    (void*)&nred, (void*)&a.part, (void*)&a.ctr, (void*)&sa};
    hipError_t e = hipLaunchKernel(fn, dim3(groups), dim3(64 * krk::kStreamWaves), args, shm, stream);
    return hip_status(e, "stream_gemm_kernel launch");
}

template <int MT, bool SILU, bool XF = false>
int dispatch_stream_xs(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    const int xs = stream_xs(MT, cdiv(cdiv(a.K, krk::kStreamKC), c.splits));
    if constexpr (MT == 1) {
        switch (xs) {
            case 4: return launch_stream<1, 4, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 5: return launch_stream<1, 5, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 8: return launch_stream<1, 8, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 10: return launch_stream<1, 10, SILU, 0, XF>(a, nblocks, c.unroll, s);
        }
    } else if constexpr (MT == 2) {
        switch (xs) {
            case 4: return launch_stream<2, 4, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 5: return launch_stream<2, 5, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 8: return launch_stream<2, 8, SILU, 0, XF>(a, nblocks, c.unroll, s);
        }
    } else {
        switch (xs) {
            case 4: return launch_stream<MT, 4, SILU, 0, XF>(a, nblocks, c.unroll, s);
            case 5: return launch_stream<MT, 5, SILU, 0, XF>(a, nblocks, c.unroll, s);
        }
    }
    return fail(KRK_ERR_UNSUPPORTED, "STREAM has no x-register layout for m_tiles=%d and this K split", MT);
}

// The selection epilogue of the stream kernel is instantiated for K in 5
// stages (the hidden size 2560 the lm_head reads), K unsplit: argmax at every
// M, top-kSelMaxK up to 16 rows.  Measured (lm_head): the running top-8 lists
// add 3.5 us to the projection at M <= 16, against 6.4 us saved by reading
// keys instead of logits; at 32 rows they add 11.6 us, more than they save.
constexpr int kStreamSelStages = 5;
constexpr int kStreamTopkMaxTiles = 1;

template <int SK>
int dispatch_stream_sel(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s,
                        const krk::SelectArgs& sa) {
    if (c.m_tiles == 1) return launch_stream<1, kStreamSelStages, false, SK>(a, nblocks, c.unroll, s, sa);
    if constexpr (SK == 1) {
        switch (c.m_tiles) {
            case 2: return launch_stream<2, kStreamSelStages, false, 1>(a, nblocks, c.unroll, s, sa);
            case 3: return launch_stream<3, kStreamSelStages, false, 1>(a, nblocks, c.unroll, s, sa);
            case 4: return launch_stream<4, kStreamSelStages, false, 1>(a, nblocks, c.unroll, s, sa);
        }
    }
    return fail(KRK_ERR_UNSUPPORTED, "STREAM selection epilogue: m_tiles=%d", c.m_tiles);
}

// xf: x in the kernel's fragment order (a normed call's prologue wrote it).
template <bool SILU>
int dispatch_stream(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s, bool xf = false) {
    switch (c.m_tiles) {
        case 1: return xf ? dispatch_stream_xs<1, SILU, true>(a, c, nblocks, s) : dispatch_stream_xs<1, SILU>(a, c, nblocks, s);
        case 2: return xf ? dispatch_stream_xs<2, SILU, true>(a, c, nblocks, s) : dispatch_stream_xs<2, SILU>(a, c, nblocks, s);
        case 3: return xf ? dispatch_stream_xs<3, SILU, true>(a, c, nblocks, s) : dispatch_stream_xs<3, SILU>(a, c, nblocks, s);
        case 4: return xf ? dispatch_stream_xs<4, SILU, true>(a, c, nblocks, s) : dispatch_stream_xs<4, SILU>(a, c, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "STREAM m_tiles=%d", c.m_tiles);
}

template <int KC, int NT, int NGV, int XGV, int D>
int launch_slice(const LaunchArgs& a, int nblocks, hipStream_t stream) {
    constexpr int MT = cdiv_c(XGV * krk::slice_rg(KC), 16);
    const void* fn = reinterpret_cast<const void*>(&krk::slice_gemm_kernel<MT, NT, D, KC, NGV, XGV>);
    const size_t shm = krk::slice_lds_bytes(MT, NT, D, NGV, XGV);
    static std::atomic<uint64_t> done{0};
    const hipError_t attr = shm > 65536 ? ensure_lds_limit(fn, (int)shm, done) : hipSuccess;
    if (attr != hipSuccess) return hip_status(attr, "slice_gemm_kernel LDS attribute");
    // Chunk ranges of the splits, so the kernel divides nothing.
    const int nch = cdiv(a.K, KC);
    int cper = nch / a.splits, crem = nch % a.splits, cb = a.cb;
    void* args[] = {(void*)&a.x, (void*)&a.ldx, (void*)&a.w,      (void*)&a.ldw, (void*)&a.y,    (void*)&a.ldy,
                    (void*)&a.M, (void*)&a.N,   (void*)&a.K,      (void*)&a.splits, (void*)&cb, (void*)&cper,
                    (void*)&crem, (void*)&a.part, (void*)&a.ctr};
    hipError_t e = hipLaunchKernel(fn, dim3(nblocks, a.splits), dim3(64 * krk::kSliceWaves), args, shm, stream);
    return hip_status(e, "slice_gemm_kernel launch");
}

template <int KC, int NT, int NGV, int XGV>
int dispatch_slice_d(const LaunchArgs& a, int D, int nblocks, hipStream_t s) {
    if (D == 2) {
        if constexpr (slice_inst(KC, NT, NGV, XGV, 2)) return launch_slice<KC, NT, NGV, XGV, 2>(a, nblocks, s);
    } else if (D == 3) {
        if constexpr (slice_inst(KC, NT, NGV, XGV, 3)) return launch_slice<KC, NT, NGV, XGV, 3>(a, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "SLICE variant KC=%d NT=%d groups %d+%d D=%d", KC, NT, NGV, XGV, D);
}

template <int KC, int NT, int NGV>
int dispatch_slice_x(const LaunchArgs& a, int XGV, int D, int nblocks, hipStream_t s) {
    switch (XGV) {
        case 1: return dispatch_slice_d<KC, NT, NGV, 1>(a, D, nblocks, s);
        case 2: return dispatch_slice_d<KC, NT, NGV, 2>(a, D, nblocks, s);
        case 3: return dispatch_slice_d<KC, NT, NGV, 3>(a, D, nblocks, s);
        case 4: return dispatch_slice_d<KC, NT, NGV, 4>(a, D, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "SLICE x groups=%d", XGV);
}

template <int KC>
int dispatch_slice_kc(const LaunchArgs& a, const SliceShape& v, int D, int nblocks, hipStream_t s) {
    if (v.NT == 1) {
        switch (v.NGV) {
            case 1: return dispatch_slice_x<KC, 1, 1>(a, v.XGV, D, nblocks, s);
            case 2: return dispatch_slice_x<KC, 1, 2>(a, v.XGV, D, nblocks, s);
            case 3: return dispatch_slice_x<KC, 1, 3>(a, v.XGV, D, nblocks, s);
            case 4: return dispatch_slice_x<KC, 1, 4>(a, v.XGV, D, nblocks, s);
        }
    } else if (v.NT == 2) {
        switch (v.NGV) {
            case 3: return dispatch_slice_x<KC, 2, 3>(a, v.XGV, D, nblocks, s);
            case 4: return dispatch_slice_x<KC, 2, 4>(a, v.XGV, D, nblocks, s);
        }
    }
    return fail(KRK_ERR_UNSUPPORTED, "SLICE weight tiles=%d groups=%d", v.NT, v.NGV);
}

int dispatch_slice(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    const SliceShape v = slice_shape(c.k_chunk, a.cb, a.M);
    return c.k_chunk == 128 ? dispatch_slice_kc<128>(a, v, c.unroll, nblocks, s)
                            : dispatch_slice_kc<64>(a, v, c.unroll, nblocks, s);
}

template <int MX, int R, int D, bool SILU, bool NORM = false, bool SEL = false>
int launch_valu(const LaunchArgs& a, int nblocks, int waves, hipStream_t stream, krk::NormArgs na = {},
                krk::SelectArgs sa = {}) {
    const int nb = cdiv(a.K, krk::kValuBlock);
    int per = nb / a.splits, rem = nb % a.splits;
    // Whole 512-element blocks and whole D-block chunks in every split: the
    // kernel variant without clamps or masks.
    const bool exact = a.K % krk::kValuBlock == 0 && rem == 0 && per % D == 0;
    const void* fn = exact ? reinterpret_cast<const void*>(&krk::valu_gemm_kernel<MX, R, D, SILU, true, NORM, SEL>)
                           : reinterpret_cast<const void*>(&krk::valu_gemm_kernel<MX, R, D, SILU, false, NORM, SEL>);
    const size_t shm = NORM ? krk::valu_norm_lds_bytes(MX, nb) : krk::valu_lds_bytes(MX, cdiv(nb, a.splits));
    if (NORM || MX >= krk::kValuLdsMinRows) {
        static std::atomic<uint64_t> done[2] = {{0}, {0}};
        const hipError_t attr = ensure_lds_limit(fn, (int)kLdsMax, done[exact]);
        if (attr != hipSuccess) return hip_status(attr, "valu_gemm_kernel LDS attribute");
    }
    void* args[] = {(void*)&a.x, (void*)&a.ldx, (void*)&a.w, (void*)&a.ldw, (void*)&a.y,    (void*)&a.ldy, (void*)&a.M,
                    (void*)&a.N, (void*)&a.K,   (void*)&per, (void*)&rem, (void*)&a.part, (void*)&a.ctr, (void*)&na, (void*)&sa};
    hipError_t e = hipLaunchKernel(fn, dim3(nblocks, a.splits), dim3(64 * waves), args, shm, stream);
    return hip_status(e, "valu_gemm_kernel launch");
}

template <int MX, int R, int D, bool SILU>
int launch_valu_if(const LaunchArgs& a, int nblocks, int waves, hipStream_t s) {
    constexpr int loads = (MX < krk::kValuLdsMinRows ? MX + R : R) * D;
    if constexpr (loads <= 48) {
        return launch_valu<MX, R, D, SILU>(a, nblocks, waves, s);
    } else {
        return fail(KRK_ERR_UNSUPPORTED, "VALU unroll=%d with %d rows per wave", D, R);
    }
}

template <int MX, int R, bool SILU>
int dispatch_valu_d(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    switch (c.unroll) {
        case 2: return launch_valu_if<MX, R, 2, SILU>(a, nblocks, c.waves, s);
        case 3: return launch_valu_if<MX, R, 3, SILU>(a, nblocks, c.waves, s);
        case 4: return launch_valu_if<MX, R, 4, SILU>(a, nblocks, c.waves, s);
        case 5: return launch_valu_if<MX, R, 5, SILU>(a, nblocks, c.waves, s);
        case 7: return launch_valu_if<MX, R, 7, SILU>(a, nblocks, c.waves, s);
        case 8: return launch_valu_if<MX, R, 8, SILU>(a, nblocks, c.waves, s);
        case 10: return launch_valu_if<MX, R, 10, SILU>(a, nblocks, c.waves, s);
        case 19: return launch_valu_if<MX, R, 19, SILU>(a, nblocks, c.waves, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "VALU unroll=%d with %d rows per wave", c.unroll, R);
}

template <int MX, bool SILU>
int dispatch_valu_r(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    if constexpr (!SILU) {
        if (c.n_tiles == 1) return dispatch_valu_d<MX, 1, false>(a, c, nblocks, s);
    }
    if (c.n_tiles == 2) return dispatch_valu_d<MX, 2, SILU>(a, c, nblocks, s);
    if (c.n_tiles == 4) return dispatch_valu_d<MX, 4, SILU>(a, c, nblocks, s);
    return fail(KRK_ERR_UNSUPPORTED, "VALU n_tiles=%d", c.n_tiles);
}

template <bool SILU>
int dispatch_valu(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s) {
    switch (c.m_tiles) {
        case 1: return dispatch_valu_r<1, SILU>(a, c, nblocks, s);
        case 2: return dispatch_valu_r<2, SILU>(a, c, nblocks, s);
        case 4: return dispatch_valu_r<4, SILU>(a, c, nblocks, s);
        case 8: return dispatch_valu_r<8, SILU>(a, c, nblocks, s);
    }
    return fail(KRK_ERR_UNSUPPORTED, "VALU x rows=%d", c.m_tiles);
}

// The fused RMSNorm prologue is instantiated for the VALU depth that covers a
// K of 2560 (the hidden size every normed projection reads) in one pass.
constexpr int kValuNormDepth = 5;

template <int MX, bool SILU>
int dispatch_valu_norm_r(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s,
                         const krk::NormArgs& na) {
    if constexpr (!SILU) {
        if (c.n_tiles == 1) return launch_valu<MX, 1, kValuNormDepth, false, true>(a, nblocks, c.waves, s, na);
    }
    if (c.n_tiles == 2) return launch_valu<MX, 2, kValuNormDepth, SILU, true>(a, nblocks, c.waves, s, na);
    if (c.n_tiles == 4) return launch_valu<MX, 4, kValuNormDepth, SILU, true>(a, nblocks, c.waves, s, na);
    return fail(KRK_ERR_UNSUPPORTED, "VALU n_tiles=%d", c.n_tiles);
}

template <bool SILU>
int dispatch_valu_norm(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s,
                       const krk::NormArgs& na) {
    switch (c.m_tiles) {
        case 1: return dispatch_valu_norm_r<1, SILU>(a, c, nblocks, s, na);
        case 2: return dispatch_valu_norm_r<2, SILU>(a, c, nblocks, s, na);
        case 4: return dispatch_valu_norm_r<4, SILU>(a, c, nblocks, s, na);
        case 8: return dispatch_valu_norm_r<8, SILU>(a, c, nblocks, s, na);
    }
    return fail(KRK_ERR_UNSUPPORTED, "VALU normed: x rows=%d", c.m_tiles);
}

// The LDS-staged kernel with the fused prologue: 512-k stages, K unsplit, one
// or two 16-row x tiles and one or two weight tiles (the normalised rows of
// all stages stay in registers); with two of each, three stages in flight
// would spill, so that pair runs two.
constexpr int kLdsNormMaxMTiles = 2;
constexpr int kLdsNormMaxNTiles = 2;
constexpr bool lds_norm_pf3(int MT, int NT) { return MT == 1 || NT == 1; }

template <int MT, int NT, bool SILU>
int dispatch_mfma_lds_norm_pf(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s,
                              const krk::NormArgs& na) {
    if constexpr (lds_norm_pf3(MT, NT)) {
        if (c.unroll == 3) return launch_mfma_lds<MT, NT, 3, 512, SILU, false, true>(a, nblocks, s, {}, na);
    }
    return launch_mfma_lds<MT, NT, 2, 512, SILU, false, true>(a, nblocks, s, {}, na);
}

template <bool SILU>
int dispatch_mfma_lds_norm(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s,
                           const krk::NormArgs& na) {
    if constexpr (!SILU) {
        if (c.m_tiles == 1 && c.n_tiles == 1) return dispatch_mfma_lds_norm_pf<1, 1, false>(a, c, nblocks, s, na);
        if (c.m_tiles == 2 && c.n_tiles == 1) return dispatch_mfma_lds_norm_pf<2, 1, false>(a, c, nblocks, s, na);
    }
    if (c.m_tiles == 1 && c.n_tiles == 2) return dispatch_mfma_lds_norm_pf<1, 2, SILU>(a, c, nblocks, s, na);
    if (c.m_tiles == 2 && c.n_tiles == 2) return dispatch_mfma_lds_norm_pf<2, 2, SILU>(a, c, nblocks, s, na);
    return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS normed: m_tiles=%d n_tiles=%d", c.m_tiles, c.n_tiles);
}

// Whether a resolved configuration fuses the RMSNorm prologue into the
// projection kernel (one launch), else a separate prologue kernel writes the
// normalised rows first (also what prologue = 1 asks for).  Both keep the
// reference's rounding points (krk_norm.h).  Fused, with K unsplit:
//   * a VALU configuration at the depth covering K = 2560, with a wave per
//     512-k block (M <= 8);
//   * an LDS-staged MFMA configuration with 512-k stages, K <= 2560, one or
//     two x tiles and one or two weight tiles, two stages in flight when
//     both are two (M <= 32; the reference offers its fused prologue up to
//     M = 32, engine/kernels/gemm.py:524-531).
//
// Every workgroup of a fused call normalises all M rows itself (about ten
// VALU instructions per element), so the fused form pays only at small M:
// measured on MI355X, normed qkv / gate_up / lm_head at M = 1 take 7.2 /
// 16.8 / 106.9 us fused against 9.7 / 19.6 / 110.6 us behind the prologue
// kernel, while at M = 4 gate_up takes 22.7 us fused against 20.6 us.  (A
// fused form of the persistent stream kernel never beat the prologue kernel:
// each of its 256 workgroups normalises every row, ~3 us per 16 rows of
// VALU work ahead of the first MFMA.)
bool norm_fused(int M, int N, int K, int epilogue, const krk_gemm_config& c) {
    (void)M;
    (void)N;
    (void)epilogue;
    if (c.prologue != 0 || c.splits != 1) return false;
    const int nb = cdiv(K, krk::kValuBlock);
    if (c.kernel == KRK_KERNEL_MFMA_LDS)
        return c.k_chunk == 512 && nb <= krk::kLdsNormStages && c.m_tiles <= kLdsNormMaxMTiles &&
               c.n_tiles <= kLdsNormMaxNTiles && (c.unroll == 2 || lds_norm_pf3(c.m_tiles, c.n_tiles));
    if (c.kernel != KRK_KERNEL_VALU) return false;
    return c.unroll == kValuNormDepth && nb <= c.waves && krk::valu_norm_lds_bytes(c.m_tiles, nb) <= kLdsMax;
}

// Plans of the normed calls (cfg == NULL): fused configurations where they
// measured fastest (tuner, graph replay over rotating weights, MI355X); every
// other shape and M runs its plain plan behind the prologue kernel.
const TableEntry kNormTable[] = {
    // qkv: 256 workgroups of 6 waves x 4 rows.  From M = 5 the prologue
    // kernel + the wave-sliced plain plan (0.1-0.4 us under the LDS-staged
    // kernel's fused form at M = 6-16, even at M = 5, in four runs).
    {6144, 2560, KRK_EPILOGUE_NONE, 1, 4, kcfg(KRK_KERNEL_VALU, 4, 5, 6, 1)},
    {19456, 2560, KRK_EPILOGUE_SILU_MUL, 1, 2, kcfg(KRK_KERNEL_VALU, 2, 5, 8, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 1, 1, kcfg(KRK_KERNEL_VALU, 1, 5, 8, 1)},
    {151936, 2560, KRK_EPILOGUE_NONE, 2, 2, kcfg(KRK_KERNEL_VALU, 2, 5, 8, 1)},
};

int normed_plan(int M, int N, int K, int epilogue, krk_gemm_config* out) {
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    for (const TableEntry& e : kNormTable)
        if (e.N == N && e.K == K && e.epilogue == epilogue && Mc >= e.m_lo && Mc <= e.m_hi)
            return resolve_config(M, N, K, epilogue, &e.cfg, out);
    const int rc = resolve_config(M, N, K, epilogue, nullptr, out);
    if (rc == KRK_OK) out->prologue = 1;
    return rc;
}

// A normed call's configuration: the caller's, else the normed plan.
int resolve_normed(int M, int N, int K, int epilogue, const krk_gemm_config* cfg, krk_gemm_config* out) {
    return cfg ? resolve_config(M, N, K, epilogue, cfg, out) : normed_plan(M, N, K, epilogue, out);
}

// The residual-add + RMSNorm prologue of a normed call (krk_norm.h).
struct NormSpec {
    const void* d;
    int64_t ldd;
    const void* w_norm;
    float eps;
    void* xout;
    int64_t ldxo;
};

// A normed call whose projection runs on the stream kernel in one launch
// gets its normalised rows in that kernel's fragment order.  (The same
// handover to the LDS-staged kernel with x in registers, its tiles then
// holding weight rows only, measured no faster: normed qkv at M = 17-32
// 12.8-12.9 against 12.3-12.9 us behind the row-major prologue.)
inline bool frag_prologue(int M, const krk_gemm_config& c) {
    return c.kernel == KRK_KERNEL_STREAM && M <= kMaxRowsPerLaunch;
}

// Workspace of a call: [split-K counters and partials][normalised rows
// when a separate prologue writes them: M x K bf16, or in the stream
// kernel's fragment order, 16·m_tiles rows x whole 512-k stages].
struct WorkspaceLayout {
    size_t gemm;   // split-K part, at offset 0
    size_t n_off;  // offset of the normalised rows (0 if none)
    size_t total;
};
WorkspaceLayout workspace_layout(int M, int N, int K, int epilogue, const krk_gemm_config& c, bool normed) {
    WorkspaceLayout l;
    l.gemm = workspace_for(M, N, epilogue, c);
    const bool prologue = normed && !norm_fused(M, N, K, epilogue, c);
    const size_t nbytes = frag_prologue(M, c) ? krk::frag_bytes(c.m_tiles, K) : (size_t)M * K * sizeof(uint16_t);
    l.n_off = prologue ? align_up(l.gemm, 256) : 0;
    l.total = prologue ? l.n_off + nbytes : l.gemm;
    return l;
}

// fixed_part_off: 0 for the caller-sized workspace layout; otherwise the
// split-K partials start at this offset and the counters of every call share
// the region before it (the allocation-free entry point's static scratch).
int gemm_impl(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
              int M, int N, int K, int epilogue, const krk_gemm_config* cfg,
              void* workspace, size_t workspace_bytes, void* stream, const NormSpec* ns = nullptr,
              size_t fixed_part_off = 0) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    if (!x || !w || !y) return fail(KRK_ERR_INVALID, "null operand pointer (x=%p w=%p y=%p)", x, w, y);
    const bool silu = epilogue == KRK_EPILOGUE_SILU_MUL;
    const int Nout = silu ? N / 2 : N;
    if (ldx < K || ldw < K) return fail(KRK_ERR_INVALID, "ldx=%lld / ldw=%lld must be >= K=%d", (long long)ldx, (long long)ldw, K);
    if (ldy < Nout) return fail(KRK_ERR_INVALID, "ldy=%lld must be >= %d output columns", (long long)ldy, Nout);
    if ((ldx % 8) || (ldw % 8)) return fail(KRK_ERR_ALIGN, "ldx=%lld and ldw=%lld must be multiples of 8 elements", (long long)ldx, (long long)ldw);
    if (((uintptr_t)x % 16) || ((uintptr_t)w % 16)) return fail(KRK_ERR_ALIGN, "x=%p and w=%p must be 16-byte aligned", x, w);
    if ((uintptr_t)y % 2) return fail(KRK_ERR_ALIGN, "y=%p must be 2-byte aligned", y);
    if (ns) {
        if (!ns->d || !ns->w_norm || !ns->xout)
            return fail(KRK_ERR_INVALID, "null norm operand (d=%p w_norm=%p xout=%p)", ns->d, ns->w_norm, ns->xout);
        if (ns->ldd < K || ns->ldxo < K)
            return fail(KRK_ERR_INVALID, "ldd=%lld / ldxo=%lld must be >= K=%d", (long long)ns->ldd, (long long)ns->ldxo, K);
        if ((ns->ldd % 8) || (ns->ldxo % 8))
            return fail(KRK_ERR_ALIGN, "ldd=%lld and ldxo=%lld must be multiples of 8 elements", (long long)ns->ldd, (long long)ns->ldxo);
        if (((uintptr_t)ns->d % 16) || ((uintptr_t)ns->w_norm % 16) || ((uintptr_t)ns->xout % 16))
            return fail(KRK_ERR_ALIGN, "d, w_norm and xout must be 16-byte aligned");
        if (!(ns->eps >= 0.0f) || ns->eps == __builtin_inff())
            return fail(KRK_ERR_INVALID, "eps=%g must be finite and >= 0", (double)ns->eps);
        if (K > krk::kNormThreads * 8 * krk::kNormMaxVec)
            return fail(KRK_ERR_UNSUPPORTED, "the RMSNorm prologue handles K <= %d, got %d",
                        krk::kNormThreads * 8 * krk::kNormMaxVec, K);
    }

    krk_gemm_config c;
    rc = ns ? resolve_normed(M, N, K, epilogue, cfg, &c) : resolve_config(M, N, K, epilogue, cfg, &c);
    if (rc) return rc;

    const uintptr_t x0 = (uintptr_t)x, x1 = x0 + ((uint64_t)(M - 1) * ldx + K) * 2;
    const uintptr_t w0 = (uintptr_t)w, w1 = w0 + ((uint64_t)(N - 1) * ldw + K) * 2;
    const uintptr_t y0 = (uintptr_t)y, y1 = y0 + ((uint64_t)(M - 1) * ldy + Nout) * 2;
    if (overlaps(y0, y1, x0, x1) || overlaps(y0, y1, w0, w1))
        return fail(KRK_ERR_ALIAS, "output y may not share memory with x or W");
    uintptr_t o0 = 0, o1 = 0;
    if (ns) {
        // Every workgroup reads all of x and d while one of them writes xout,
        // so xout may share memory with none of the operands.
        o0 = (uintptr_t)ns->xout;
        o1 = o0 + ((uint64_t)(M - 1) * ns->ldxo + K) * 2;
        const uintptr_t d0 = (uintptr_t)ns->d, d1 = d0 + ((uint64_t)(M - 1) * ns->ldd + K) * 2;
        const uintptr_t g0 = (uintptr_t)ns->w_norm, g1 = g0 + (uint64_t)K * 2;
        if (overlaps(o0, o1, x0, x1) || overlaps(o0, o1, d0, d1) || overlaps(o0, o1, g0, g1) ||
            overlaps(o0, o1, w0, w1) || overlaps(o0, o1, y0, y1))
            return fail(KRK_ERR_ALIAS, "xout may not share memory with x, d, w_norm, W or y");
        if (overlaps(y0, y1, d0, d1) || overlaps(y0, y1, g0, g1))
            return fail(KRK_ERR_ALIAS, "output y may not share memory with d or w_norm");
    }

    const WorkspaceLayout wl = workspace_layout(M, N, K, epilogue, c, ns != nullptr);
    if (wl.total) {
        if (!workspace) return fail(KRK_ERR_WORKSPACE, "this plan needs a %zu-byte workspace, got none", wl.total);
        if (workspace_bytes < wl.total)
            return fail(KRK_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes, wl.total);
        if ((uintptr_t)workspace % 16) return fail(KRK_ERR_ALIGN, "workspace=%p must be 16-byte aligned", workspace);
        const uintptr_t s0 = (uintptr_t)workspace, s1 = s0 + wl.total;
        if (overlaps(s0, s1, x0, x1) || overlaps(s0, s1, w0, w1) || overlaps(s0, s1, y0, y1) ||
            (ns && overlaps(s0, s1, o0, o1)))
            return fail(KRK_ERR_ALIAS, "workspace may not share memory with x, W, y or xout");
    }

    const Geometry g = geometry(M, N, epilogue, c);
    uint32_t* ctr = wl.gemm ? static_cast<uint32_t*>(workspace) : nullptr;
    const size_t part_off = fixed_part_off ? fixed_part_off : align_up((size_t)g.nblocks * sizeof(uint32_t), 256);
    float* part = wl.gemm ? reinterpret_cast<float*>(static_cast<char*>(workspace) + part_off) : nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    krk::NormArgs na{};
    if (ns) na = krk::NormArgs{static_cast<const uint16_t*>(ns->d), ns->ldd, static_cast<const uint16_t*>(ns->w_norm),
                               ns->eps, static_cast<uint16_t*>(ns->xout), ns->ldxo};
    const bool fused = ns && norm_fused(M, N, K, epilogue, c);
    // Projection input: x itself, or the normalised rows a prologue kernel
    // writes into the workspace.
    const uint16_t* xin = static_cast<const uint16_t*>(x);
    int64_t ldin = ldx;
    const bool xf = ns && !fused && frag_prologue(M, c);
    if (xf) {
        unsigned char* nf = static_cast<unsigned char*>(workspace) + wl.n_off;
        int mt = c.m_tiles;
        void* args[] = {(void*)&x, (void*)&ldx, (void*)&na, (void*)&nf, (void*)&M, (void*)&K, (void*)&mt};
        hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&krk::add_rmsnorm_frag_kernel), dim3(16 * mt),
                                       dim3(krk::kNormThreads), args, 0, st);
        if ((rc = hip_status(e, "add_rmsnorm_frag_kernel launch"))) return rc;
        xin = reinterpret_cast<const uint16_t*>(nf);
        ldin = 0;  // unused: the fragment order has no row stride
    } else if (ns && !fused) {
        uint16_t* nrows = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + wl.n_off);
        int64_t ldn = K;
        void* args[] = {(void*)&x, (void*)&ldx, (void*)&na, (void*)&nrows, (void*)&ldn, (void*)&K};
        hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&krk::add_rmsnorm_kernel), dim3(M),
                                       dim3(krk::kNormThreads), args, 0, st);
        if ((rc = hip_status(e, "add_rmsnorm_kernel launch"))) return rc;
        xin = nrows;
        ldin = ldn;
    }
    for (int m0 = 0; m0 < M; m0 += kMaxRowsPerLaunch) {
        LaunchArgs a;
        a.x = xin + (int64_t)m0 * ldin;
        a.ldx = ldin;
        a.w = static_cast<const uint16_t*>(w);
        a.ldw = ldw;
        a.y = static_cast<uint16_t*>(y) + (int64_t)m0 * ldy;
        a.ldy = ldy;
        a.M = (M - m0) < kMaxRowsPerLaunch ? (M - m0) : kMaxRowsPerLaunch;
        a.N = N;
        a.K = K;
        a.splits = c.splits;
        a.part = part;
        a.ctr = ctr;
        a.cb = g.cb;
        if (fused) {
            // This chunk's rows of d and xout.
            krk::NormArgs nc = na;
            nc.d += (int64_t)m0 * na.ldd;
            nc.xout += (int64_t)m0 * na.ldxo;
            if (c.kernel == KRK_KERNEL_MFMA_LDS)
                rc = silu ? dispatch_mfma_lds_norm<true>(a, c, g.nblocks, st, nc)
                          : dispatch_mfma_lds_norm<false>(a, c, g.nblocks, st, nc);
            else
                rc = silu ? dispatch_valu_norm<true>(a, c, g.nblocks, st, nc)
                          : dispatch_valu_norm<false>(a, c, g.nblocks, st, nc);
        } else if (c.kernel == KRK_KERNEL_MFMA) {
            rc = silu ? dispatch_mfma<true>(a, c, g.nblocks, st) : dispatch_mfma<false>(a, c, g.nblocks, st);
        } else if (c.kernel == KRK_KERNEL_MFMA_LDS) {
            rc = silu ? dispatch_mfma_lds<true>(a, c, g.nblocks, st) : dispatch_mfma_lds<false>(a, c, g.nblocks, st);
        } else if (c.kernel == KRK_KERNEL_STREAM) {
            rc = silu ? dispatch_stream<true>(a, c, g.nblocks, st, xf) : dispatch_stream<false>(a, c, g.nblocks, st, xf);
        } else if (c.kernel == KRK_KERNEL_SLICE) {
            rc = dispatch_slice(a, c, g.nblocks, st);
        } else {
            rc = silu ? dispatch_valu<true>(a, c, g.nblocks, st) : dispatch_valu<false>(a, c, g.nblocks, st);
        }
        if (rc) return rc;
    }
    return KRK_OK;
}

// ----------------------------------------------------------------- token selection
// The lm_head projection followed by per-row argmax / top-k (krk_select.h).
// Two plans:
//   * fused (argmax behind a VALU, LDS-staged MFMA or stream projection, and
//     top-k behind a stream projection of up to 16 rows, K unsplit): the
//     projection's epilogue writes one key (top-k: kSelMaxK keys) per row and
//     workgroup and select_rows_kernel reduces those keys; the logits are
//     written only when the caller asks for them;
//   * unfused (top-k, and other projection plans): the plain projection
//     writes the bf16 logits (to y, or to the workspace when y is null) and
//     select_rows_kernel reduces them.
// A top-k in the epilogue was measured and rejected: its per-workgroup
// cross-lane rounds added 15-60% to the short projection workgroups, more
// than the logits' round trip through HBM costs.
constexpr int kSelValuMaxRows = 4;

template <int MX>
int dispatch_valu_sel(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s, const krk::SelectArgs& sa) {
    if (c.n_tiles == 1) return launch_valu<MX, 1, kValuNormDepth, false, false, true>(a, nblocks, c.waves, s, {}, sa);
    if (c.n_tiles == 2) return launch_valu<MX, 2, kValuNormDepth, false, false, true>(a, nblocks, c.waves, s, {}, sa);
    if (c.n_tiles == 4) return launch_valu<MX, 4, kValuNormDepth, false, false, true>(a, nblocks, c.waves, s, {}, sa);
    return fail(KRK_ERR_UNSUPPORTED, "VALU n_tiles=%d", c.n_tiles);
}

template <int MT>
int dispatch_mfma_lds_sel(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t s, const krk::SelectArgs& sa) {
    const bool pf3 = c.unroll == 3;
    if (c.n_tiles == 2) return pf3 ? launch_mfma_lds<MT, 2, 3, 256, false, true>(a, nblocks, s, sa)
                                   : launch_mfma_lds<MT, 2, 2, 256, false, true>(a, nblocks, s, sa);
    if (c.n_tiles == 4) return pf3 ? launch_mfma_lds<MT, 4, 3, 256, false, true>(a, nblocks, s, sa)
                                   : launch_mfma_lds<MT, 4, 2, 256, false, true>(a, nblocks, s, sa);
    return fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS n_tiles=%d", c.n_tiles);
}

int dispatch_plain(const LaunchArgs& a, const krk_gemm_config& c, int nblocks, hipStream_t st) {
    switch (c.kernel) {
        case KRK_KERNEL_MFMA: return dispatch_mfma<false>(a, c, nblocks, st);
        case KRK_KERNEL_MFMA_LDS: return dispatch_mfma_lds<false>(a, c, nblocks, st);
        case KRK_KERNEL_STREAM: return dispatch_stream<false>(a, c, nblocks, st);
        case KRK_KERNEL_SLICE: return dispatch_slice(a, c, nblocks, st);
        default: return dispatch_valu<false>(a, c, nblocks, st);
    }
}

// Whether argmax runs fused behind this projection plan (rows per launch Mc).
bool select_fusable(const krk_gemm_config& c, int Mc, int K, int k) {
    if (c.splits != 1) return false;
    if (c.kernel == KRK_KERNEL_STREAM)
        return cdiv(K, krk::kStreamKC) == kStreamSelStages && (k == 1 || c.m_tiles <= kStreamTopkMaxTiles);
    if (k != 1) return false;
    if (c.kernel == KRK_KERNEL_VALU) return c.m_tiles <= kSelValuMaxRows && c.unroll == kValuNormDepth;
    if (c.kernel == KRK_KERNEL_MFMA_LDS)
        return c.k_chunk == 256 && (c.n_tiles == 2 || c.n_tiles == 4) && c.m_tiles >= cdiv(Mc, 16) &&
               (c.unroll == 2 || (c.unroll == 3 && mfma_lds_pf3(c.m_tiles, c.n_tiles)));
    return false;
}

struct SelectPlan {
    krk_gemm_config c;
    bool fused;
};

// Ring depth of the plan's stream kernel when it selects tokens: the
// selecting variants keep their running keys in registers and measured
// fastest with 5 stages (lm_head M = 5-16: 116 against 119 µs for argmax,
// 122 against 131 µs for top-8 with the 7 the plain plan uses).
constexpr int kStreamSelDepth = 5;

int select_plan_for(int M, int N, int K, int k, const krk_gemm_config* cfg, SelectPlan* out) {
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    int rc = resolve_config(M, N, K, KRK_EPILOGUE_NONE, cfg, &out->c);
    if (rc) return rc;
    out->fused = select_fusable(out->c, Mc, K, k);
    if (!cfg && out->fused && out->c.kernel == KRK_KERNEL_STREAM && out->c.unroll > kStreamSelDepth)
        out->c.unroll = kStreamSelDepth;
    return KRK_OK;
}

// Workspace of a selecting call, for one launch of Mc rows (launches of a
// call run in order on one stream and reuse it):
//   [row counters, 128 B apart][projection split-K area][keys [Mc, ldk] u64 (fused)
//    or logits [Mc, ldl] bf16 (unfused; unused when the caller passes y)]
//   [chunk lists [Mc, C, k]]
struct SelectLayout {
    size_t proj, src, lists, total;
    int64_t ld;  // row stride of the source in elements
    int n;       // source elements per row
    int chunks;  // select_rows_kernel chunks per row
};
SelectLayout select_layout(int M, int N, int k, const SelectPlan& p) {
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    SelectLayout l;
    l.proj = (size_t)krk::kSelMaxRows * krk::kSelCtrStride * sizeof(uint32_t);
    size_t at = align_up(l.proj + workspace_for(Mc, N, KRK_EPILOGUE_NONE, p.c), 256);
    l.src = at;
    if (p.fused) {
        // One key per row and projection workgroup (the stream kernel's
        // workgroups each cover many blocks).
        const int nb = geometry(Mc, N, KRK_EPILOGUE_NONE, p.c).nblocks;
        l.n = p.c.kernel == KRK_KERNEL_STREAM ? stream_groups(nb, 1) * (k == 1 ? 1 : krk::kSelMaxK) : nb;
        l.ld = align_up((size_t)l.n, 2);
        at += align_up((size_t)Mc * l.ld * sizeof(uint64_t), 256);
        l.chunks = cdiv(l.n, krk::kSelChunkKeys);
    } else {
        l.n = N;
        l.ld = align_up((size_t)N, 8);
        at += align_up((size_t)Mc * l.ld * sizeof(uint16_t), 256);
        l.chunks = cdiv(N, krk::kSelChunkVals);
    }
    l.lists = at;
    at += align_up((size_t)Mc * l.chunks * k * sizeof(uint64_t), 256);
    l.total = at;
    return l;
}

template <int KM, bool KEYS>
int launch_select_rows(const krk::RowSelectArgs& ra, int chunks, int rows, hipStream_t st) {
    void* args[] = {(void*)&ra};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&krk::select_rows_kernel<KM, KEYS>), dim3(chunks, rows),
                                   dim3(krk::kSelThreads), args, 0, st);
    return hip_status(e, "select_rows_kernel launch");
}

int select_impl(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int M, int N, int K,
                int k, int64_t* idx, void* vals, const krk_gemm_config* cfg, void* workspace, size_t workspace_bytes,
                void* stream) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, KRK_EPILOGUE_NONE);
    if (rc) return rc;
    if (k < 1 || k > krk::kSelMaxK || k > N) return fail(KRK_ERR_INVALID, "k=%d must be in 1..min(%d, N)", k, krk::kSelMaxK);
    if (!x || !w || !idx) return fail(KRK_ERR_INVALID, "null operand pointer (x=%p w=%p idx=%p)", x, w, idx);
    if (ldx < K || ldw < K) return fail(KRK_ERR_INVALID, "ldx=%lld / ldw=%lld must be >= K=%d", (long long)ldx, (long long)ldw, K);
    if ((ldx % 8) || (ldw % 8)) return fail(KRK_ERR_ALIGN, "ldx=%lld and ldw=%lld must be multiples of 8 elements", (long long)ldx, (long long)ldw);
    if (((uintptr_t)x % 16) || ((uintptr_t)w % 16)) return fail(KRK_ERR_ALIGN, "x=%p and w=%p must be 16-byte aligned", x, w);
    if ((uintptr_t)idx % 8 || (uintptr_t)vals % 2 || (uintptr_t)y % 2) return fail(KRK_ERR_ALIGN, "idx, vals or y misaligned");
    if (y && ldy < N) return fail(KRK_ERR_INVALID, "ldy=%lld must be >= N=%d", (long long)ldy, N);
    SelectPlan p;
    if ((rc = select_plan_for(M, N, K, k, cfg, &p))) return rc;
    const SelectLayout l = select_layout(M, N, k, p);

    const uintptr_t x0 = (uintptr_t)x, x1 = x0 + ((uint64_t)(M - 1) * ldx + K) * 2;
    const uintptr_t w0 = (uintptr_t)w, w1 = w0 + ((uint64_t)(N - 1) * ldw + K) * 2;
    const uintptr_t i0 = (uintptr_t)idx, i1 = i0 + (uint64_t)M * k * 8;
    const uintptr_t v0 = (uintptr_t)vals, v1 = vals ? v0 + (uint64_t)M * k * 2 : v0;
    const uintptr_t y0 = (uintptr_t)y, y1 = y ? y0 + ((uint64_t)(M - 1) * ldy + N) * 2 : y0;
    const uintptr_t s0 = (uintptr_t)workspace;
    const uintptr_t s1 = s0 + l.total;
    struct Span { uintptr_t a, b; } outs[] = {{i0, i1}, {v0, v1}, {y0, y1}, {s0, s1}};
    for (int q0 = 0; q0 < 4; ++q0) {
        if (outs[q0].a == outs[q0].b) continue;
        if (overlaps(outs[q0].a, outs[q0].b, x0, x1) || overlaps(outs[q0].a, outs[q0].b, w0, w1))
            return fail(KRK_ERR_ALIAS, "outputs and workspace may not share memory with x or W");
        for (int q = q0 + 1; q < 4; ++q)
            if (outs[q].a != outs[q].b && overlaps(outs[q0].a, outs[q0].b, outs[q].a, outs[q].b))
                return fail(KRK_ERR_ALIAS, "idx, vals, y and the workspace may not overlap");
    }
    if (!workspace) return fail(KRK_ERR_WORKSPACE, "token selection needs a %zu-byte workspace, got none", l.total);
    if (workspace_bytes < l.total) return fail(KRK_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes, l.total);
    if ((uintptr_t)workspace % 256) return fail(KRK_ERR_ALIGN, "workspace=%p must be 256-byte aligned", workspace);

    hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    const Geometry g = geometry(M, N, KRK_EPILOGUE_NONE, p.c);
    for (int m0 = 0; m0 < M; m0 += kMaxRowsPerLaunch) {
        LaunchArgs a;
        a.x = static_cast<const uint16_t*>(x) + (int64_t)m0 * ldx;
        a.ldx = ldx;
        a.w = static_cast<const uint16_t*>(w);
        a.ldw = ldw;
        a.M = (M - m0) < kMaxRowsPerLaunch ? (M - m0) : kMaxRowsPerLaunch;
        a.N = N;
        a.K = K;
        a.splits = p.c.splits;
        a.ctr = p.c.splits > 1 ? reinterpret_cast<uint32_t*>(ws + l.proj) : nullptr;
        a.cb = g.cb;
        a.part = p.c.splits > 1 ? reinterpret_cast<float*>(ws + l.proj + align_up((size_t)g.nblocks * sizeof(uint32_t), 256))
                                : nullptr;
        krk::RowSelectArgs ra;
        ra.n = l.n;
        ra.ctr = reinterpret_cast<uint32_t*>(ws);
        ra.lists = reinterpret_cast<uint64_t*>(ws + l.lists);
        ra.idx = idx + (int64_t)m0 * k;
        ra.vals = vals ? static_cast<uint16_t*>(vals) + (int64_t)m0 * k : nullptr;
        ra.k = k;
        if (p.fused) {
            a.y = y ? static_cast<uint16_t*>(y) + (int64_t)m0 * ldy : nullptr;
            a.ldy = ldy;
            const krk::SelectArgs sa{reinterpret_cast<uint64_t*>(ws + l.src), l.ld};
            if (p.c.kernel == KRK_KERNEL_STREAM) {
                rc = k == 1 ? dispatch_stream_sel<1>(a, p.c, g.nblocks, st, sa)
                            : dispatch_stream_sel<krk::kSelMaxK>(a, p.c, g.nblocks, st, sa);
            } else if (p.c.kernel == KRK_KERNEL_VALU) {
                switch (p.c.m_tiles) {
                    case 1: rc = dispatch_valu_sel<1>(a, p.c, g.nblocks, st, sa); break;
                    case 2: rc = dispatch_valu_sel<2>(a, p.c, g.nblocks, st, sa); break;
                    case 4: rc = dispatch_valu_sel<4>(a, p.c, g.nblocks, st, sa); break;
                    default: rc = fail(KRK_ERR_UNSUPPORTED, "VALU x rows=%d", p.c.m_tiles);
                }
            } else {
                switch (p.c.m_tiles) {
                    case 1: rc = dispatch_mfma_lds_sel<1>(a, p.c, g.nblocks, st, sa); break;
                    case 2: rc = dispatch_mfma_lds_sel<2>(a, p.c, g.nblocks, st, sa); break;
                    case 3: rc = dispatch_mfma_lds_sel<3>(a, p.c, g.nblocks, st, sa); break;
                    case 4: rc = dispatch_mfma_lds_sel<4>(a, p.c, g.nblocks, st, sa); break;
                    default: rc = fail(KRK_ERR_UNSUPPORTED, "MFMA_LDS m_tiles=%d", p.c.m_tiles);
                }
            }
            if (rc) return rc;
            ra.src = sa.keys;
            ra.ld = l.ld;
            ra.vec = 1;
            rc = k == 1 ? launch_select_rows<1, true>(ra, l.chunks, a.M, st)
                        : launch_select_rows<krk::kSelMaxK, true>(ra, l.chunks, a.M, st);
        } else {
            uint16_t* logits = y ? static_cast<uint16_t*>(y) + (int64_t)m0 * ldy : reinterpret_cast<uint16_t*>(ws + l.src);
            a.y = logits;
            a.ldy = y ? ldy : l.ld;
            if ((rc = dispatch_plain(a, p.c, g.nblocks, st))) return rc;
            ra.src = logits;
            ra.ld = a.ldy;
            ra.vec = (a.ldy % 8 == 0) && ((uintptr_t)logits % 16 == 0);
            rc = k == 1 ? launch_select_rows<1, false>(ra, l.chunks, a.M, st)
                        : launch_select_rows<krk::kSelMaxK, false>(ra, l.chunks, a.M, st);
        }
        if (rc) return rc;
    }
    return KRK_OK;
}

// ------------------------------------------------------- allocation-free calls
// krk_gemm_bf16_noalloc keeps its split-K workspace in this static device
// array instead of a caller's buffer: counters in the first
// KRK_NOALLOC_COUNTER_BYTES (each call's blocks use counters from index 0;
// every call leaves the ones it used at zero), fp32 partials after them.  In
// host code `scratch` names a host-side stand-in, never the device memory:
// the device address comes from hipGetSymbolAddress, once per device.
constexpr int kScratchMaxDevices = 64;
std::atomic<uintptr_t> g_scratch[kScratchMaxDevices];

__global__ void zero_words_kernel(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[KRK_NOALLOC_SCRATCH_BYTES];

namespace {

// The current device's copy of `scratch`.  The first call on a device looks
// up its address and zeroes the counter region with a kernel on `stream`
// (the array starts zeroed; the clear keeps that invariant independent of the
// loader).
int scratch_on_current_device(unsigned char** out, hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kScratchMaxDevices)
        return fail(KRK_ERR_UNSUPPORTED, "device %d: the static scratch is tracked for devices 0..%d", dev,
                    kScratchMaxDevices - 1);
    uintptr_t p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        void* sym = nullptr;
        e = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
        uint32_t* ctr = static_cast<uint32_t*>(sym);
        int n = (int)(KRK_NOALLOC_COUNTER_BYTES / sizeof(uint32_t));
        void* args[] = {(void*)&ctr, (void*)&n};
        e = hipLaunchKernel(reinterpret_cast<const void*>(&zero_words_kernel), dim3(16), dim3(256), args, 0, stream);
        if (e != hipSuccess) return hip_status(e, "scratch counter clear launch");
        p = reinterpret_cast<uintptr_t>(sym);
        g_scratch[dev].store(p, std::memory_order_release);
    }
    *out = reinterpret_cast<unsigned char*>(p);
    return KRK_OK;
}

}  // namespace

extern "C" {

int krk_gemm_bf16(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                  int M, int N, int K, int epilogue, void* workspace, size_t workspace_bytes, void* stream) {
    return gemm_impl(x, ldx, w, ldw, y, ldy, M, N, K, epilogue, nullptr, workspace, workspace_bytes, stream);
}

int krk_gemm_bf16_config(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                         int M, int N, int K, int epilogue, const krk_gemm_config* cfg,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return gemm_impl(x, ldx, w, ldw, y, ldy, M, N, K, epilogue, cfg, workspace, workspace_bytes, stream);
}

int krk_gemm_bf16_normed(const void* x, int64_t ldx, const void* d, int64_t ldd, const void* w_norm, float eps,
                         void* xout, int64_t ldxo, const void* w, int64_t ldw, void* y, int64_t ldy,
                         int M, int N, int K, int epilogue, void* workspace, size_t workspace_bytes, void* stream) {
    const NormSpec ns{d, ldd, w_norm, eps, xout, ldxo};
    return gemm_impl(x, ldx, w, ldw, y, ldy, M, N, K, epilogue, nullptr, workspace, workspace_bytes, stream, &ns);
}

int krk_gemm_bf16_normed_config(const void* x, int64_t ldx, const void* d, int64_t ldd, const void* w_norm, float eps,
                                void* xout, int64_t ldxo, const void* w, int64_t ldw, void* y, int64_t ldy,
                                int M, int N, int K, int epilogue, const krk_gemm_config* cfg,
                                void* workspace, size_t workspace_bytes, void* stream) {
    const NormSpec ns{d, ldd, w_norm, eps, xout, ldxo};
    return gemm_impl(x, ldx, w, ldw, y, ldy, M, N, K, epilogue, cfg, workspace, workspace_bytes, stream, &ns);
}

size_t krk_gemm_normed_workspace_bytes(int M, int N, int K, int epilogue, const krk_gemm_config* cfg) {
    if (check_shape(M, N, K, epilogue)) return 0;
    krk_gemm_config c;
    if (resolve_normed(M, N, K, epilogue, cfg, &c)) return 0;
    return workspace_layout(M, N, K, epilogue, c, true).total;
}

int krk_gemm_normed_fused(int M, int N, int K, int epilogue, const krk_gemm_config* cfg) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    krk_gemm_config c;
    if ((rc = resolve_normed(M, N, K, epilogue, cfg, &c))) return rc;
    return norm_fused(M, N, K, epilogue, c) ? 1 : 0;
}

int krk_gemm_normed_plan(int M, int N, int K, int epilogue, krk_gemm_config* out) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    if (!out) return fail(KRK_ERR_INVALID, "null output configuration");
    return normed_plan(M, N, K, epilogue, out);
}

int krk_add_rms_norm_bf16(const void* x, int64_t ldx, const void* d, int64_t ldd, const void* w_norm, float eps,
                          void* xout, int64_t ldxo, void* out, int64_t ldo, int M, int K, void* stream) {
    g_err[0] = '\0';
    if (M < 1 || K < 8 || K % 8) return fail(KRK_ERR_INVALID, "shape M=%d K=%d: need M >= 1, K >= 8, K %% 8 == 0", M, K);
    if (K > krk::kNormThreads * 8 * krk::kNormMaxVec)
        return fail(KRK_ERR_UNSUPPORTED, "add_rms_norm handles K <= %d, got %d", krk::kNormThreads * 8 * krk::kNormMaxVec, K);
    if (!x || !d || !w_norm || !xout || !out) return fail(KRK_ERR_INVALID, "null operand pointer");
    if (ldx < K || ldd < K || ldxo < K || ldo < K) return fail(KRK_ERR_INVALID, "row strides must be >= K=%d", K);
    if ((ldx | ldd | ldxo | ldo) % 8) return fail(KRK_ERR_ALIGN, "row strides must be multiples of 8 elements");
    if (((uintptr_t)x | (uintptr_t)d | (uintptr_t)w_norm | (uintptr_t)xout | (uintptr_t)out) % 16)
        return fail(KRK_ERR_ALIGN, "operands must be 16-byte aligned");
    if (!(eps >= 0.0f) || eps == __builtin_inff()) return fail(KRK_ERR_INVALID, "eps=%g must be finite and >= 0", (double)eps);
    auto span = [&](const void* p, int64_t ld) {
        const uintptr_t a = (uintptr_t)p;
        return std::pair<uintptr_t, uintptr_t>(a, a + ((uint64_t)(M - 1) * ld + K) * 2);
    };
    const auto X = span(x, ldx), D = span(d, ldd), XO = span(xout, ldxo), O = span(out, ldo);
    const uintptr_t g0 = (uintptr_t)w_norm, g1 = g0 + (uint64_t)K * 2;
    // Each row is read and written by one workgroup, each element by one
    // thread, so xout may be x itself (the reference's in-place form).
    const bool in_place = xout == x && ldxo == ldx;
    if ((!in_place && overlaps(XO.first, XO.second, X.first, X.second)) || overlaps(XO.first, XO.second, D.first, D.second) ||
        overlaps(XO.first, XO.second, g0, g1) || overlaps(O.first, O.second, X.first, X.second) ||
        overlaps(O.first, O.second, D.first, D.second) || overlaps(O.first, O.second, g0, g1))
        return fail(KRK_ERR_ALIAS, "xout and out may not share memory with x (except xout == x), d or w_norm");
    if (overlaps(XO.first, XO.second, O.first, O.second)) return fail(KRK_ERR_ALIAS, "xout and out may not overlap");
    krk::NormArgs na{static_cast<const uint16_t*>(d), ldd, static_cast<const uint16_t*>(w_norm), eps,
                     static_cast<uint16_t*>(xout), ldxo};
    void* args[] = {(void*)&x, (void*)&ldx, (void*)&na, (void*)&out, (void*)&ldo, (void*)&K};
    hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&krk::add_rmsnorm_kernel), dim3(M),
                                   dim3(krk::kNormThreads), args, 0, static_cast<hipStream_t>(stream));
    return hip_status(e, "add_rmsnorm_kernel launch");
}

int krk_gemm_bf16_select(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                         int M, int N, int K, int k, int64_t* idx, void* vals,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return select_impl(x, ldx, w, ldw, y, ldy, M, N, K, k, idx, vals, nullptr, workspace, workspace_bytes, stream);
}

int krk_gemm_bf16_select_config(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                                int M, int N, int K, int k, int64_t* idx, void* vals, const krk_gemm_config* cfg,
                                void* workspace, size_t workspace_bytes, void* stream) {
    return select_impl(x, ldx, w, ldw, y, ldy, M, N, K, k, idx, vals, cfg, workspace, workspace_bytes, stream);
}

size_t krk_gemm_select_workspace_bytes(int M, int N, int K, int k, const krk_gemm_config* cfg) {
    if (check_shape(M, N, K, KRK_EPILOGUE_NONE) || k < 1 || k > krk::kSelMaxK || k > N) return 0;
    SelectPlan p;
    if (select_plan_for(M, N, K, k, cfg, &p)) return 0;
    return select_layout(M, N, k, p).total;
}

int krk_gemm_select_plan(int M, int N, int K, int k, krk_gemm_config* out) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, KRK_EPILOGUE_NONE);
    if (rc) return rc;
    if (k < 1 || k > krk::kSelMaxK || k > N) return fail(KRK_ERR_INVALID, "k=%d must be in 1..min(%d, N)", k, krk::kSelMaxK);
    if (!out) return fail(KRK_ERR_INVALID, "null output config");
    SelectPlan p;
    if ((rc = select_plan_for(M, N, K, k, nullptr, &p))) return rc;
    *out = p.c;
    return KRK_OK;
}

int krk_gemm_select_fused(int M, int N, int K, int k, const krk_gemm_config* cfg) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, KRK_EPILOGUE_NONE);
    if (rc) return rc;
    if (k < 1 || k > krk::kSelMaxK || k > N) return fail(KRK_ERR_INVALID, "k=%d must be in 1..min(%d, N)", k, krk::kSelMaxK);
    SelectPlan p;
    if ((rc = select_plan_for(M, N, K, k, cfg, &p))) return rc;
    return p.fused ? 1 : 0;
}

int krk_gemm_bf16_noalloc(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
                          int M, int N, int K, int epilogue, void* stream) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    krk_gemm_config c;
    auto_config(M, N, K, epilogue, &c);
    if (c.splits > 1) {
        const Geometry g = geometry(M, N, epilogue, c);
        const size_t counters = (size_t)g.nblocks * sizeof(uint32_t);
        const size_t partials = (size_t)c.splits * (size_t)g.Mc * (size_t)N * sizeof(float);
        if (counters > KRK_NOALLOC_COUNTER_BYTES || partials > KRK_NOALLOC_SCRATCH_BYTES - KRK_NOALLOC_COUNTER_BYTES)
            return fail(KRK_ERR_WORKSPACE,
                        "M=%d N=%d K=%d: the plan splits K %d ways and needs %zu bytes of partials and %d counters; "
                        "the static scratch holds %zu bytes of partials and %zu counters (use krk_gemm_bf16 with a "
                        "workspace)", M, N, K, c.splits, partials, g.nblocks,
                        (size_t)(KRK_NOALLOC_SCRATCH_BYTES - KRK_NOALLOC_COUNTER_BYTES),
                        (size_t)(KRK_NOALLOC_COUNTER_BYTES / sizeof(uint32_t)));
    }
    unsigned char* s = nullptr;
    if ((rc = scratch_on_current_device(&s, static_cast<hipStream_t>(stream)))) return rc;
    return gemm_impl(x, ldx, w, ldw, y, ldy, M, N, K, epilogue, nullptr, s, KRK_NOALLOC_SCRATCH_BYTES, stream, nullptr,
                     KRK_NOALLOC_COUNTER_BYTES);
}

size_t krk_gemm_workspace_bytes(int M, int N, int K, int epilogue) {
    if (check_shape(M, N, K, epilogue)) return 0;
    krk_gemm_config c;
    auto_config(M, N, K, epilogue, &c);
    return workspace_for(M, N, epilogue, c);
}

size_t krk_gemm_config_workspace_bytes(int M, int N, int K, int epilogue, const krk_gemm_config* cfg) {
    if (check_shape(M, N, K, epilogue)) return 0;
    krk_gemm_config c;
    if (resolve_config(M, N, K, epilogue, cfg, &c)) return 0;
    return workspace_for(M, N, epilogue, c);
}

int krk_gemm_resolve(int M, int N, int K, int epilogue, const krk_gemm_config* cfg, krk_gemm_config* out) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    if (!out) return fail(KRK_ERR_INVALID, "null output config");
    return resolve_config(M, N, K, epilogue, cfg, out);
}

int krk_gemm_plan(int M, int N, int K, int epilogue, krk_gemm_config* out) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    if (!out) return fail(KRK_ERR_INVALID, "null output config");
    auto_config(M, N, K, epilogue, out);
    return KRK_OK;
}

int krk_gemm_candidates(int M, int N, int K, int epilogue, krk_gemm_config* out, int cap) {
    g_err[0] = '\0';
    int rc = check_shape(M, N, K, epilogue);
    if (rc) return rc;
    if (cap < 0 || (cap > 0 && !out)) return fail(KRK_ERR_INVALID, "need an output array for cap=%d configurations", cap);
    const int Mc = M < kMaxRowsPerLaunch ? M : kMaxRowsPerLaunch;
    constexpr int kMax = 1024;
    krk_gemm_config found[kMax];
    int n = 0;
    auto add = [&](const krk_gemm_config& want) {
        krk_gemm_config r;
        if (resolve_config(M, N, K, epilogue, &want, &r)) return;
        for (int i = 0; i < n; ++i)
            if (!memcmp(&found[i], &r, sizeof r)) return;
        if (n < kMax) found[n++] = r;
    };
    krk_gemm_config plan;
    auto_config(M, N, K, epilogue, &plan);
    add(plan);
    const int nts[] = {1, 2, 4};
    const int splits[] = {1, 2, 3, 4};
    // VALU: unroll 0 covers a split's K range in one pass; 2 and 4 blocks in
    // flight per row leave more waves resident (fewer VGPRs).  5 and 6 waves
    // cut some grids to exactly one workgroup per CU (o: 2560 channels = 256
    // workgroups of 5 waves x 2 rows; qkv: 6144 = 256 x 6 waves x 4 rows).
    if (Mc <= kValuMaxRows)
        for (int nt : nts)
            for (int wv : {4, 5, 6, krk::kValuMaxWaves})
                for (int sp : splits)
                    for (int u : {0, 2, 4}) add(krk_gemm_config{KRK_KERNEL_VALU, 0, nt, u, wv, sp, 0});
    // More splits for the weight-streaming MFMA kernels: at M >= 16 they cut
    // each workgroup's share of x, the bound of narrow-N, long-K shapes.
    const int wide_splits[] = {1, 2, 3, 4, 6, 8};
    // LDS-staged: every tile width, each with all its channels and with
    // fewer (the rest of the last tile padding), so a grid can match the CUs
    // (qkv: 256 blocks of 24 channels).
    for (int nt : nts) {
        const int full = 16 * (epilogue == KRK_EPILOGUE_SILU_MUL ? nt / 2 : nt);
        const int chans[] = {full, full - 8, full * 5 / 8 / 8 * 8, full / 2};
        for (int pf : {2, 3})
            for (int kc : {256, 512})
                for (int sp : wide_splits)
                    for (int ch : chans)
                        if (ch >= 8) add(krk_gemm_config{KRK_KERNEL_MFMA_LDS, 0, nt, pf, 0, sp, kc, 0, ch, 1});
        // x held in registers for the whole K (one K split, 512-k stages).
        for (int pf : {2, 3})
            for (int ch : chans)
                if (ch >= 8) add(krk_gemm_config{KRK_KERNEL_MFMA_LDS, 0, nt, pf, 0, 1, 512, 0, ch, 2});
    }
    for (int d = 2; d <= krk::kStreamMaxDepth; ++d)
        for (int sp : wide_splits) add(krk_gemm_config{KRK_KERNEL_STREAM, 0, 0, d, 0, sp, 0});
    for (int nt : nts)
        for (int sp : {1, 2, 4}) add(krk_gemm_config{KRK_KERNEL_MFMA, 0, nt, 4, 4, sp, 0});
    // SLICE: one block per CU (per CU and split), the same rounded up to 8,
    // and whole 16-row tiles; 64- and 128-k chunks, 2 or 3 in flight.
    if (epilogue == KRK_EPILOGUE_NONE && Mc <= kSliceMaxRows)
        for (int sp : {1, 2})
            for (int kc : {64, 128})
                for (int d : {2, 3}) {
                    const int one = cdiv(N * sp, kCuCount);
                    for (int ch : {one, cdiv(one, 8) * 8, 16, 32})
                        add(krk_gemm_config{KRK_KERNEL_SLICE, 0, 0, d, 0, sp, kc, 0, ch, 0});
                }
    g_err[0] = '\0';  // rejected candidates are not an error of this call
    for (int i = 0; i < n && i < cap; ++i) out[i] = found[i];
    return n;
}

const char* krk_last_error(void) { return g_err; }

int krk_abi_version(void) { return KRK_ABI_VERSION; }

size_t krk_gemm_config_size(void) { return sizeof(krk_gemm_config); }

}  // extern "C"
