// thermal.hip -- EQ3 RC thermal grid and the thermal-coupled reliability
// run for gfx950 (MI355X).
//
// k_thermal_window advances the grid by one backward-Euler step
// (thermal.cpp:127-160 on a regular 6-neighbour network) with `sweeps`
// Jacobi sweeps, temporally blocked: a workgroup stages its tile plus a halo
// of `sweeps` cells in LDS, sweeps there, and writes only the interior, whose
// values are exact after the last sweep.  HBM traffic per step is one read
// and one write of the temperature (plus the power array when it is given).
// In coupled mode the same launch first runs the window's control,
// retention and refresh decisions (every workgroup computes them for all
// dies, workgroup 0 stores them), builds the cell power from the window's
// per-die access counts, and after the step folds every die's hotspot into
// the next row of the hotspot trace with atomic maxima.
//
// Floating-point contraction is off in this file: every cell's update is the
// same sequence of IEEE double operations as the CPU restatement, so
// temperatures, hotspots and every decision derived from them are
// bit-identical to it.
#include <hip/hip_runtime.h>

#include "thermal.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <type_traits>
#include <vector>

#pragma clang fp contract(off)

namespace hbfamd {
namespace {

constexpr int kThreads = 256;  // workgroups of the admission-gate and gather kernels
constexpr int kCellsPerThread = 8;
// Staged tile regions: up to kMaxRegion cells, or kMaxWideRegion for the
// wide tiles of big uncoupled grids (65.5 KB of LDS for the two sweep
// buffers, two workgroups per CU), whose halo re-reads fewer cells per owned
// cell (14 x 14 interiors in 22 x 22 regions at 8 layers: 2.5x, against 4x
// for 8 x 8 interiors in 16 x 16 regions).
constexpr std::uint32_t kMaxRegion = 2048;
constexpr std::uint32_t kMaxWideRegion = 4096;
// Tiles are swept by 512-thread workgroups: 2-4 cells per thread, 8 for wide
// regions.  Against 256 threads with up to 8 cells each, the extra waves
// hide the sweeps' LDS latency (the coupled 64 x 64 x 8 grid: 8.2 -> 6.6 us
// per window).
constexpr int kTileBlock = 512;
static_assert(kMaxWideRegion == kTileBlock * kCellsPerThread, "wide region");
constexpr std::uint32_t kAfBins = 4096;
constexpr double kAfT0 = 200.0;
constexpr double kAfStepsPerK = 16.0;
constexpr std::uint32_t kNoPending = 4;
constexpr std::uint32_t kMaxDies = 1024;

struct Ctl {
    std::uint32_t applied;
    std::uint32_t pending;
    std::uint64_t pending_at;
    std::uint64_t last_change;
};

struct TArgs {
    std::uint32_t nx, ny, nz, sweeps;
    std::uint32_t tx, ty, rx, ry;  // tile interior and staged region
    std::uint32_t tiles_x;
    std::uint32_t block;           // threads per workgroup (kTileBlock)
    std::uint32_t cells;           // rx * ry * nz
    std::uint32_t step_x, step_y, step_z;  // 256 in the region's mixed radix
    double cdt, gx, gy, gz, gb, tb;
    const double* power;           // W per cell (uncoupled steps)
    // coupled mode
    std::uint32_t coupled;
    std::uint32_t ndie, regions_x, rw, rh, lpd, D;
    double static_w, pa, pr;
    const std::uint32_t* counts;   // [windows][ndie]
    unsigned long long* hot;       // [(windows + 1)][ndie], bits of doubles
    const std::uint64_t* af;       // retention table
    std::uint64_t retention_ps, window_ps;
    const std::uint64_t* age_in;
    std::uint64_t* age_out;
    std::uint8_t* refresh;
    // non-null in a captured chunk of windows: the window index is this
    // counter plus the launch's own offset in the chunk
    const std::uint64_t* wbase;
};

__device__ __forceinline__ std::uint64_t sat_add(std::uint64_t a, std::uint64_t b)
{
    return a > ~0ull - b ? ~0ull : a + b;
}

__device__ __forceinline__ std::uint32_t af_bin(double t)
{
    if (!(t >= kAfT0)) {
        return 0;
    }
    const double f = (t - kAfT0) * kAfStepsPerK;
    if (!(f < static_cast<double>(kAfBins - 1))) {
        return kAfBins - 1;
    }
    return static_cast<std::uint32_t>(f);
}

// Neighbour bits of a staged cell: which neighbours exist in the grid
// (update terms) and which of those are staged in LDS.
enum : std::uint32_t {
    kIn = 1u << 0,
    kXm = 1u << 1, kXmL = 1u << 2, kXp = 1u << 3, kXpL = 1u << 4,
    kYm = 1u << 5, kYmL = 1u << 6, kYp = 1u << 7, kYpL = 1u << 8,
    kZm = 1u << 9, kZp = 1u << 10, kTop = 1u << 11, kInterior = 1u << 12
};

template <bool kCoupled, int kCells, int kBlock = kTileBlock>
__global__ __launch_bounds__(kBlock) void k_thermal_window(TArgs a, const double* tin,
                                                             double* tout, std::uint64_t w)
{
    // LDS: cur[cells + 1] and nxt[cells + 1]; slot `cells` of both holds
    // 0.0 and stands for every neighbour outside the grid.
    extern __shared__ double lds[];
    __shared__ std::uint8_t s_ref[kCoupled ? kMaxDies : 1];
    __shared__ unsigned long long s_hot[kCoupled ? 64 : 1];
    if (kCoupled && a.wbase != nullptr) {
        w += *a.wbase;
    }
    const std::uint32_t rx = a.rx, ry = a.ry, nz = a.nz, nx = a.nx, ny = a.ny;
    const std::uint32_t cells = a.cells, plane = rx * ry, sweeps = a.sweeps;
    const std::uint32_t tx = a.tx, ty = a.ty, h = sweeps;
    const std::uint32_t zero = cells;
    double* cur = lds;
    double* nxt = lds + cells + 1;
    const int tid = threadIdx.x;
    const std::uint32_t tile_x = blockIdx.x % a.tiles_x;
    const std::uint32_t tile_y = blockIdx.x / a.tiles_x;
    const int x0 = static_cast<int>(tile_x * tx) - static_cast<int>(h);
    const int y0 = static_cast<int>(tile_y * ty) - static_cast<int>(h);
    const double cdt = a.cdt, gx = a.gx, gy = a.gy, gz = a.gz, gb = a.gb;
    const double gbtb = gb * a.tb;

    // 1. Owned cells c = tid + 256 k.  Per cell, once: its grid index, die,
    //    the LDS slots of its six neighbours (`zero` outside the grid; the
    //    cell itself outside the staged region, which disturbs only cells
    //    within `sweeps` of the region edge), 1 / den with den summed in the
    //    CPU restatement's order, and its ambient term.  The grid index and
    //    die come first (1a), so that the window's global loads (2) are in
    //    flight while the rest (1b, with its divisions) is computed.
    std::uint32_t gidx[kCells], die[kCells], fl[kCells];
    std::uint32_t cx[kCells], cy[kCells], cz[kCells];
    std::uint32_t nbr[kCells][6];
    double rden[kCells], topv[kCells];
    std::uint32_t safe_die = 0;
    {
        std::uint32_t xi = static_cast<std::uint32_t>(tid) % rx;
        std::uint32_t t0 = static_cast<std::uint32_t>(tid) / rx;
        std::uint32_t yi = t0 % ry;
        std::uint32_t zi = t0 / ry;
        // The tile lies inside one channel-way region; its halo reaches at
        // most one region further (sweeps <= region size, checked on the
        // host), so a cell's region differs from the tile's by -1, 0 or 1.
        int qx0 = 0, qy0 = 0, rx0 = 0, ry0 = 0;
        if (kCoupled) {
            qx0 = static_cast<int>((tile_x * tx) / a.rw);
            qy0 = static_cast<int>((tile_y * ty) / a.rh);
            rx0 = qx0 * static_cast<int>(a.rw);
            ry0 = qy0 * static_cast<int>(a.rh);
            safe_die = (static_cast<std::uint32_t>(qy0) * a.regions_x +
                        static_cast<std::uint32_t>(qx0)) * a.D;
        }
#pragma unroll
        for (int k = 0; k < kCells; ++k) {
            const std::uint32_t c = tid + k * kBlock;
            const int gxx = x0 + static_cast<int>(xi);
            const int gyy = y0 + static_cast<int>(yi);
            std::uint32_t f = 0, g = 0, d = safe_die;
            if (c < cells && gxx >= 0 && gxx < static_cast<int>(nx) && gyy >= 0 &&
                gyy < static_cast<int>(ny)) {
                g = (zi * ny + static_cast<std::uint32_t>(gyy)) * nx + static_cast<std::uint32_t>(gxx);
                f = kIn;
                if (xi >= h && xi < h + tx && yi >= h && yi < h + ty) f |= kInterior;
                if (kCoupled) {
                    const int qx = qx0 + (gxx < rx0 ? -1 : (gxx >= rx0 + static_cast<int>(a.rw) ? 1 : 0));
                    const int qy = qy0 + (gyy < ry0 ? -1 : (gyy >= ry0 + static_cast<int>(a.rh) ? 1 : 0));
                    d = (static_cast<std::uint32_t>(qy) * a.regions_x +
                         static_cast<std::uint32_t>(qx)) * a.D + zi / a.lpd;
                }
            }
            fl[k] = f;
            gidx[k] = g;
            die[k] = d;
            cx[k] = xi;
            cy[k] = yi;
            cz[k] = zi;
            xi += a.step_x;
            const std::uint32_t carry_x = xi >= rx ? 1u : 0u;
            xi -= carry_x * rx;
            yi += a.step_y + carry_x;
            const std::uint32_t carry_y = yi >= ry ? 1u : 0u;
            yi -= carry_y * ry;
            zi += a.step_z + carry_y;
        }
    }
    // 2. Every independent global load at once (cells outside the grid load
    //    index 0 and are masked).
    double v[kCells], pin[kCells];
    std::uint32_t cnt[kCells];
#pragma unroll
    for (int k = 0; k < kCells; ++k) {
        v[k] = tin[gidx[k]];
        if (kCoupled) {
            cnt[k] = a.counts[w * a.ndie + die[k]];
        } else {
            pin[k] = a.power[gidx[k]];
        }
    }
    // 1b. Neighbour slots, 1 / den and the ambient term.
#pragma unroll
    for (int k = 0; k < kCells; ++k) {
        const std::uint32_t c = tid + k * kBlock;
        const std::uint32_t xi = cx[k], yi = cy[k], zi = cz[k];
        const int gxx = x0 + static_cast<int>(xi);
        const int gyy = y0 + static_cast<int>(yi);
        std::uint32_t n0 = zero, n1 = zero, n2 = zero, n3 = zero, n4 = zero, n5 = zero;
        double den = cdt, top = 0.0;
        if (fl[k] & kIn) {
            if (gxx > 0) { n0 = xi > 0 ? c - 1 : c; den += gx; }
            if (gxx + 1 < static_cast<int>(nx)) { n1 = xi + 1 < rx ? c + 1 : c; den += gx; }
            if (gyy > 0) { n2 = yi > 0 ? c - rx : c; den += gy; }
            if (gyy + 1 < static_cast<int>(ny)) { n3 = yi + 1 < ry ? c + rx : c; den += gy; }
            if (zi > 0) { n4 = c - plane; den += gz; }
            if (zi + 1 < nz) {
                n5 = c + plane;
                den += gz;
            } else {
                den += gb;
                top = gbtb;
            }
        }
        nbr[k][0] = n0; nbr[k][1] = n1; nbr[k][2] = n2;
        nbr[k][3] = n3; nbr[k][4] = n4; nbr[k][5] = n5;
        rden[k] = (fl[k] & kIn) ? 1.0 / den : 0.0;
        topv[k] = top;
    }
    if (kCoupled) {
        // this window's retention and refresh decisions for every die (all
        // blocks; block 0 stores them)
        const double* hrow = reinterpret_cast<const double*>(a.hot + w * a.ndie);
        for (std::uint32_t d = tid; d < a.ndie; d += kBlock) {
            std::uint64_t age = a.age_in[d];
            if (w > 0) {
                age = sat_add(age, a.af[af_bin(hrow[d])]);
            }
            const std::uint8_t rf = age >= a.retention_ps ? 1 : 0;
            if (rf) {
                age = 0;
            }
            s_ref[d] = rf;
            if (blockIdx.x == 0) {
                a.age_out[d] = age;
                a.refresh[w * a.ndie + d] = rf;
            }
        }
        if (tid < 64) {
            s_hot[tid] = 0;
        }
        __syncthreads();
    }

    // 3. Right-hand sides C/dt T + P and the staged temperatures.
    double rhs[kCells];
#pragma unroll
    for (int k = 0; k < kCells; ++k) {
        const std::uint32_t c = tid + k * kBlock;
        double p;
        if (kCoupled) {
            p = (a.static_w + static_cast<double>(cnt[k]) * a.pa) +
                static_cast<double>(s_ref[die[k]]) * a.pr;
        } else {
            p = pin[k];
        }
        const bool in = (fl[k] & kIn) != 0;
        rhs[k] = in ? cdt * v[k] + p : 0.0;
        if (c < cells) {
            cur[c] = in ? v[k] : 0.0;
        }
    }
    if (tid == 0) {
        cur[zero] = 0.0;
        nxt[zero] = 0.0;
    }
    __syncthreads();

    // 4. Jacobi sweeps in LDS: num accumulates the six neighbour terms in
    //    order (a neighbour outside the grid adds gx * 0.0 = +0.0, exact)
    //    and the ambient term; the update is num * (1 / den).
    for (std::uint32_t s = 0; s < sweeps; ++s) {
        double out[kCells];
#pragma unroll
        for (int k = 0; k < kCells; ++k) {
            double num = rhs[k];
            num += gx * cur[nbr[k][0]];
            num += gx * cur[nbr[k][1]];
            num += gy * cur[nbr[k][2]];
            num += gy * cur[nbr[k][3]];
            num += gz * cur[nbr[k][4]];
            num += gz * cur[nbr[k][5]];
            num += topv[k];
            out[k] = num * rden[k];
        }
#pragma unroll
        for (int k = 0; k < kCells; ++k) {
            const std::uint32_t c = tid + k * kBlock;
            if (c < cells) {
                nxt[c] = out[k];
            }
        }
        __syncthreads();
        double* t = cur;
        cur = nxt;
        nxt = t;
    }

    // 5. Interior write-back and per-die hotspots.
#pragma unroll
    for (int k = 0; k < kCells; ++k) {
        if (fl[k] & kInterior) {
            const double val = cur[tid + k * kBlock];
            tout[gidx[k]] = val;
            if (kCoupled) {
                atomicMax(&s_hot[die[k] - safe_die],
                          static_cast<unsigned long long>(__double_as_longlong(val)));
            }
        }
    }
    if (kCoupled) {
        __syncthreads();
        if (tid < static_cast<int>(a.D)) {
            atomicMax(&a.hot[(w + 1) * a.ndie + safe_die + tid], s_hot[tid]);
        }
    }
}

// Every tile launch uses kTileBlock threads (TArgs built with that block).
template <bool kCoupled>
void launch_window(const TArgs& a, std::uint32_t blocks, std::size_t lds, hipStream_t stream,
                   const double* tin, double* tout, std::uint64_t w)
{
    const std::uint32_t per = (a.cells + kTileBlock - 1) / kTileBlock;
    if (!kCoupled && per > 4) {  // wide regions of up to kMaxWideRegion cells
        hipLaunchKernelGGL((k_thermal_window<false, kCellsPerThread, kTileBlock>), dim3(blocks),
                           dim3(kTileBlock), lds, stream, a, tin, tout, w);
    } else if (per <= 2) {
        hipLaunchKernelGGL((k_thermal_window<kCoupled, 2, kTileBlock>), dim3(blocks),
                           dim3(kTileBlock), lds, stream, a, tin, tout, w);
    } else if (per <= 3) {
        hipLaunchKernelGGL((k_thermal_window<kCoupled, 3, kTileBlock>), dim3(blocks),
                           dim3(kTileBlock), lds, stream, a, tin, tout, w);
    } else {
        hipLaunchKernelGGL((k_thermal_window<kCoupled, 4, kTileBlock>), dim3(blocks),
                           dim3(kTileBlock), lds, stream, a, tin, tout, w);
    }
}

// ---- marching stencil for large uncoupled grids ----------------------------
// A workgroup owns a strip of 64 x columns (one wave per z layer, lane = x
// offset) over a segment of rows, and walks it along y.  Each row that enters
// (level 0: T and P from memory) is swept L times on the way through: S
// sweeps of one step, or 2 S when a pass makes two steps with the same
// power (the first step's result, at level S, becomes the second step's
// start and right-hand side without leaving the chip).  At step t, level k
// (1..L) updates row t - 2k from level k - 1's rows t - 2k - 1 .. t - 2k + 1,
// all of which earlier steps wrote; the z neighbours' values come from step
// t - 2, so one barrier per two steps separates every writer from its
// readers.  A thread keeps its own cell's last 4 rows of every level in
// registers (written at step s, read at s + 1 .. s + 3); the level's rows
// also go to an LDS ring of 4 for the layers above and below, which read
// them 2 steps later.  The right-hand side of a row stays in the owning
// thread's registers until its last sweep.
// Halo: L columns on each side of the W = 64 - 2L written columns, and L
// rows at each end of a segment, against L on every side of a square tile;
// the lanes and rows next to the staged edge read a stand-in (0.0 for the
// lane beyond the wave, a zero row before the segment) and only feed cells
// that are not written.  Workgroups run 64 x nz threads, so up to 16 layers.
// Cells outside the grid hold 0.0 at every level, so a missing x or y
// neighbour adds g * 0.0 = +0.0 exactly as the per-tile kernel's zero slot
// does; a missing z neighbour is read from the cell itself with conductance
// 0.0, which adds the same +0.0.
constexpr int kMarchLanes = 64;
constexpr int kMarchAhead = 4;  // rows of T and P loaded ahead of their use (= ring length)

struct MArgs {
    std::uint32_t nx, ny, nz;
    std::uint32_t strips, seg_len, total, per_xcd;
    double cdt, gx, gy, gz, gb, tb;
    const double* power;
};

// Per-thread constants of the marching kernel.
struct MCtx {
    std::size_t col;     // this thread's cell in row 0 of its layer (x clamped into the grid)
    std::uint32_t nx;
    int ny, ys, ye, tload;
    bool xin, own;
    double cdt, gx, gy, gzm, gzp, top;
    double rden0, rden1, rden2, rden3;
    double* me;          // this thread's LDS slot of level 0, ring slot 0
    const double* pzm;   // the same for the z - 1 and z + 1 neighbours (the
    const double* pzp;   // thread itself in the bottom and top layers)
};

// S sweeps per step, F steps per pass (1 or 2, the same power in both): the
// pass sweeps L = F S levels.
template <int S, int F>
struct MRows {
    static constexpr int L = S * F;
    double pt[kMarchAhead], pp[kMarchAhead];  // T and P of rows loaded ahead
    double rh[2 * S + 1];                     // rh[i]: right-hand side of row t - i
    double ph[F == 2 ? 2 * S + 1 : 1];        // ph[i]: power of row t - i (second step)
    double rh1[F == 2 ? 2 * S + 1 : 1];       // rh1[i]: second step's right-hand side of row t - 2S - i
    double h[L][4];                           // h[k][r & 3]: this cell's level k at row r
};

__device__ __forceinline__ bool march_enters(const MCtx& c, int r)
{
    return c.xin && r >= 0 && r < c.tload;
}

// Rows outside [0, tload) and lanes outside the grid load the lane's row-0
// cell (in bounds) and use 0.0 instead.
__device__ __forceinline__ std::size_t march_at(const MCtx& c, int r)
{
    return c.col + (march_enters(c, r) ? static_cast<std::size_t>(r) * c.nx : std::size_t{0});
}

// The value of the lane one below (kCtrl = wave_shr:1, 0x138) or one above
// (wave_shl:1, 0x130) in the wave; lanes 0 and 63 get 0.0 for the missing one.
template <int kCtrl>
__device__ __forceinline__ double wave_shift(double v)
{
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), kCtrl, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), kCtrl, 0xF, 0xF, true);
    return __longlong_as_double((static_cast<long long>(hi) << 32) |
                                static_cast<long long>(static_cast<unsigned>(lo)));
}

// Step t, in ring slot J = t & 3.  kInner: rows t - 2S .. t - 2 lie in
// 1 .. ny - 2 and row t enters, so no row checks are needed.  A thread keeps
// its own cell's values of every level in registers: those give the y - 1
// and y + 1 terms, and the neighbouring lanes' copies (a one-lane wave shift)
// the x - 1 and x + 1 terms; only the z neighbours, held by other waves, are
// read from LDS.
template <int S, int F, bool kInner, int J>
__device__ __forceinline__ void march_step(const MCtx& c, MRows<S, F>& m, int t, double tv,
                                           double pv, double* tout)
{
    constexpr int kRing = 4 * kMarchLanes;
    constexpr int L = S * F;
#pragma unroll
    for (int i = 2 * S; i > 0; --i) {
        m.rh[i] = m.rh[i - 1];
    }
    m.rh[0] = c.cdt * tv + pv;
    if constexpr (F == 2) {
#pragma unroll
        for (int i = 2 * S; i > 0; --i) {
            m.ph[i] = m.ph[i - 1];
            m.rh1[i] = m.rh1[i - 1];
        }
        m.ph[0] = pv;
    }
    m.h[0][J] = tv;
    c.me[J * kMarchLanes] = tv;  // level 0
#pragma unroll
    for (int k = 1; k <= L; ++k) {
        const int r = t - 2 * k;
        const int qr = (J - 2 * k) & 3;
        const double cr = m.h[k - 1][qr];
        const int sr = (k - 1) * kRing + qr * kMarchLanes;
        double num = k <= S ? m.rh[2 * k] : m.rh1[2 * (k - S)];
        num += c.gx * wave_shift<0x138>(cr);
        num += c.gx * wave_shift<0x130>(cr);
        num += c.gy * m.h[k - 1][(J - 2 * k - 1) & 3];
        num += c.gy * m.h[k - 1][(J - 2 * k + 1) & 3];
        num += c.gzm * c.pzm[sr];
        num += c.gzp * c.pzp[sr];
        num += c.top;
        double v;
        if (kInner) {
            v = num * c.rden3;
        } else {
            // (values made opaque first, so the choice stays a register select
            // rather than a load from a chosen address of the context)
            double d0 = c.rden0, d1 = c.rden1, d2 = c.rden2, d3 = c.rden3;
            asm volatile("" : "+v"(d0), "+v"(d1), "+v"(d2), "+v"(d3));
            const double rd = r > 0 ? (r + 1 < c.ny ? d3 : d1) : (r + 1 < c.ny ? d2 : d0);
            v = (r >= 0 && r < c.ny) ? num * rd : 0.0;
        }
        if constexpr (F == 2) {
            if (k == S) {  // the first step's result: the second step's T and start
                m.rh1[0] = c.cdt * v + m.ph[2 * S];
            }
        }
        if (k < L) {
            m.h[k][qr] = v;
            c.me[k * kRing + qr * kMarchLanes] = v;
        } else if (c.own && r >= c.ys && r < c.ye) {
            tout[c.col + static_cast<std::size_t>(r) * c.nx] = v;
        }
    }
}

template <int S, int F, int J>
__device__ __forceinline__ void march_sub(const MCtx& c, MRows<S, F>& m, int t, const double* tin,
                                          const double* power, double* tout)
{
    const bool ent = march_enters(c, t);
    const double tv = ent ? m.pt[J] : 0.0, pv = ent ? m.pp[J] : 0.0;
    // the next load into pt[J] / pp[J] is issued after row t's values are
    // taken (the empty asm orders them), so both rows share the registers and
    // the loop carries no copies of pending loads; it sits before the branch
    // so that both paths keep the loaded rows in the same registers (a
    // pending load in other registers on one path would make the wait
    // analysis drain every prefetched row on the other)
    std::size_t nxt = march_at(c, t + kMarchAhead);
    asm volatile("" : "+v"(nxt) : "v"(tv), "v"(pv));
    m.pt[J] = tin[nxt];
    m.pp[J] = power[nxt];
    if (t >= 2 * S * F + 1 && t < c.tload) {
        march_step<S, F, true, J>(c, m, t, tv, pv, tout);
    } else {
        march_step<S, F, false, J>(c, m, t, tv, pv, tout);
    }
    // One barrier per two steps.  Step t reads the z neighbours' level k - 1
    // of row t - 2k, written at step t - 2, so steps t and t + 1 (t even) read
    // only what the previous pair wrote; the pair reads ring slots t - 2k and
    // t - 2k + 1 of level k - 1 while writing slots t - 2k + 2 and t - 2k + 3,
    // disjoint in the 4-slot ring, and the next pair's writes to the slots
    // read here come after the barrier.
    if constexpr ((J & 1) != 0) {
        __syncthreads();
    }
}

// Threads per workgroup the marching kernel is built for: up to 16 layers
// with 1-4 sweeps, up to 8 with 5-8 (whose registers exceed 128 per lane).
__host__ __device__ constexpr int march_max_threads(int s)
{
    return s <= 4 ? 16 * kMarchLanes : 8 * kMarchLanes;
}

template <int S, int F = 1>
__global__ __launch_bounds__(march_max_threads(S * F)) void k_thermal_march(MArgs a,
                                                                            const double* tin,
                                                                            double* tout)
{
    // LDS: [z][level 0..L-1][ring slot 0..3][64 lanes], read only by the
    // layers above and below; every offset from a thread's base is a
    // compile-time constant once steps are unrolled by 4
    extern __shared__ double lds[];
    constexpr int L = S * F;  // levels: F steps of S sweeps
    constexpr int W = kMarchLanes - 2 * L;
    constexpr int kLayer = L * 4 * kMarchLanes;
    // consecutive workgroups go to different XCDs: give each XCD a run of
    // neighbouring strips, so the halo columns they share hit one L2 (and the
    // strips of a segment, walking the same rows together, read whole rows)
    const std::uint32_t b = blockIdx.x;
    const std::uint32_t id = (b % 8u) * a.per_xcd + b / 8u;
    if (id >= a.total) {
        return;  // the whole workgroup
    }
    const int lane = static_cast<int>(threadIdx.x) & (kMarchLanes - 1);
    const int z = static_cast<int>(threadIdx.x) / kMarchLanes;
    const int nx = static_cast<int>(a.nx), ny = static_cast<int>(a.ny), nz = static_cast<int>(a.nz);
    const int strip = static_cast<int>(id % a.strips);
    MCtx c;
    c.nx = a.nx;
    c.ny = ny;
    c.ys = static_cast<int>((id / a.strips) * a.seg_len);
    c.ye = c.ys + static_cast<int>(a.seg_len) < ny ? c.ys + static_cast<int>(a.seg_len) : ny;
    c.tload = c.ye + L < ny ? c.ye + L : ny;
    const int x = strip * W - L + lane;
    c.xin = x >= 0 && x < nx;
    c.own = c.xin && lane >= L && lane < kMarchLanes - L;
    c.cdt = a.cdt;
    c.gx = a.gx;
    c.gy = a.gy;
    // 1 / den for the four y cases (bit 0: row above exists, bit 1: row
    // below), den summed in the CPU restatement's order: x-, x+, y-, y+, z-,
    // then z+ or the ambient link.  0.0 for lanes outside the grid, whose
    // updates (finite num times 0.0) are then 0.0.
    double rden[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        double den = a.cdt;
        if (x > 0) den += a.gx;
        if (x + 1 < nx) den += a.gx;
        if (k & 1) den += a.gy;
        if (k & 2) den += a.gy;
        if (z > 0) den += a.gz;
        if (z + 1 < nz) {
            den += a.gz;
        } else {
            den += a.gb;
        }
        rden[k] = c.xin ? 1.0 / den : 0.0;
    }
    c.rden0 = rden[0];
    c.rden1 = rden[1];
    c.rden2 = rden[2];
    c.rden3 = rden[3];
    c.top = z + 1 < nz ? 0.0 : a.gb * a.tb;
    c.gzm = z > 0 ? a.gz : 0.0;
    c.gzp = z + 1 < nz ? a.gz : 0.0;
    c.me = lds + z * kLayer + lane;
    c.pzm = c.me - (z > 0 ? kLayer : 0);
    c.pzp = c.me + (z + 1 < nz ? kLayer : 0);
    c.col = static_cast<std::size_t>(z) * a.nx * a.ny + (c.xin ? x : 0);
#pragma unroll
    for (int k = 0; k < 4 * L; ++k) {
        c.me[k * kMarchLanes] = 0.0;
    }
    // Rows [ys - L, ye + L) enter (those inside the grid from memory).  Steps
    // start at a multiple of 4 at or before ys - L, so that row t sits in
    // ring slot t & 3 = its index in the unrolled body, and run in whole
    // rounds of 4; the extra steps only sweep rows that are not written.
    const int t0 = (c.ys - L) & ~3;
    const int t1 = t0 + ((c.ye + 2 * L - t0 + 3) & ~3);
    MRows<S, F> m;
#pragma unroll
    for (int j = 0; j < kMarchAhead; ++j) {
        m.pt[j] = tin[march_at(c, t0 + j)];
        m.pp[j] = a.power[march_at(c, t0 + j)];
    }
#pragma unroll
    for (int i = 0; i <= 2 * S; ++i) {
        m.rh[i] = 0.0;
        if constexpr (F == 2) {
            m.ph[i] = 0.0;
            m.rh1[i] = 0.0;
        }
    }
#pragma unroll
    for (int k = 0; k < L; ++k) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            m.h[k][q] = 0.0;
        }
    }
    __syncthreads();
    for (int t = t0; t < t1; t += kMarchAhead) {
        march_sub<S, F, 0>(c, m, t, tin, a.power, tout);
        march_sub<S, F, 1>(c, m, t + 1, tin, a.power, tout);
        march_sub<S, F, 2>(c, m, t + 2, tin, a.power, tout);
        march_sub<S, F, 3>(c, m, t + 3, tin, a.power, tout);
    }
}

template <int S, int F>
hipError_t launch_march_s(const MArgs& m, std::uint32_t blocks, std::uint32_t threads,
                          std::size_t lds, hipStream_t stream, const double* tin, double* tout)
{
    hipLaunchKernelGGL((k_thermal_march<S, F>), dim3(blocks), dim3(threads), lds, stream, m, tin,
                       tout);
    return hipGetLastError();
}

using MarchLaunch = hipError_t (*)(const MArgs&, std::uint32_t, std::uint32_t, std::size_t,
                                   hipStream_t, const double*, double*);

// Fused passes (F = 2) exist for 1-4 sweeps per step (up to 8 levels).
const void* march_kernel(std::uint32_t s, int f = 1)
{
    if (f == 2) {
        switch (s) {
        case 1: return reinterpret_cast<const void*>(k_thermal_march<1, 2>);
        case 2: return reinterpret_cast<const void*>(k_thermal_march<2, 2>);
        case 3: return reinterpret_cast<const void*>(k_thermal_march<3, 2>);
        case 4: return reinterpret_cast<const void*>(k_thermal_march<4, 2>);
        default: return nullptr;
        }
    }
    switch (s) {
    case 1: return reinterpret_cast<const void*>(k_thermal_march<1>);
    case 2: return reinterpret_cast<const void*>(k_thermal_march<2>);
    case 3: return reinterpret_cast<const void*>(k_thermal_march<3>);
    case 4: return reinterpret_cast<const void*>(k_thermal_march<4>);
    case 5: return reinterpret_cast<const void*>(k_thermal_march<5>);
    case 6: return reinterpret_cast<const void*>(k_thermal_march<6>);
    case 7: return reinterpret_cast<const void*>(k_thermal_march<7>);
    case 8: return reinterpret_cast<const void*>(k_thermal_march<8>);
    default: return nullptr;
    }
}

MarchLaunch march_launcher(std::uint32_t s, int f = 1)
{
    if (f == 2) {
        switch (s) {
        case 1: return launch_march_s<1, 2>;
        case 2: return launch_march_s<2, 2>;
        case 3: return launch_march_s<3, 2>;
        case 4: return launch_march_s<4, 2>;
        default: return nullptr;
        }
    }
    switch (s) {
    case 1: return launch_march_s<1, 1>;
    case 2: return launch_march_s<2, 1>;
    case 3: return launch_march_s<3, 1>;
    case 4: return launch_march_s<4, 1>;
    case 5: return launch_march_s<5, 1>;
    case 6: return launch_march_s<6, 1>;
    case 7: return launch_march_s<7, 1>;
    case 8: return launch_march_s<8, 1>;
    default: return nullptr;
    }
}

// The marching stencil takes grids of at least kMarchMinCells cells with up
// to 16 layers at 1-4 sweeps per step, up to 8 layers at 5-8 sweeps, at
// least two strips wide and eight rows per sweep long, whose rings fit the
// workgroup's LDS limit.  Returns the LDS bytes, 0 when it does not apply.
constexpr std::size_t kMarchMinCells = std::size_t{1} << 21;

// f = 2: the fused pass of two steps (2 sweeps levels), under the same rules.
std::size_t march_lds(const hbfsim_amd_thermal_grid& g, std::size_t lds_limit, int f = 1)
{
    const std::size_t cells = static_cast<std::size_t>(g.nx) * g.ny * g.nz;
    if (march_kernel(g.sweeps, f) == nullptr || g.nz > 16 || cells < kMarchMinCells) {
        return 0;
    }
    const std::uint32_t levels = g.sweeps * static_cast<std::uint32_t>(f);
    const std::uint32_t W = kMarchLanes - 2 * levels;
    const std::uint32_t threads = kMarchLanes * g.nz;
    if (threads > static_cast<std::uint32_t>(march_max_threads(static_cast<int>(levels)))) {
        return 0;
    }
    const std::size_t lds = static_cast<std::size_t>(levels) * 4 * threads * sizeof(double);
    if (lds > lds_limit || g.nx < 2 * W || g.ny < 8 * levels) {
        return 0;
    }
    return lds;
}

// Row 0 of the hotspot trace: every die's hottest cell of the initial grid.
__global__ void k_die_hot(TArgs a, const double* t, unsigned long long* row)
{
    const std::size_t n = static_cast<std::size_t>(a.nx) * a.ny * a.nz;
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
        const std::uint32_t x = static_cast<std::uint32_t>(i % a.nx);
        const std::uint32_t y = static_cast<std::uint32_t>((i / a.nx) % a.ny);
        const std::uint32_t z = static_cast<std::uint32_t>(i / (static_cast<std::size_t>(a.nx) * a.ny));
        const std::uint32_t q = (y / a.rh) * a.regions_x + x / a.rw;
        atomicMax(&row[q * a.D + z / a.lpd],
                  static_cast<unsigned long long>(__double_as_longlong(t[i])));
    }
}

// Advances a captured chunk's window counter (one thread).
__global__ void k_add_u64(std::uint64_t* p, std::uint64_t k)
{
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        p[0] += k;
    }
}

__global__ void k_fill_u64(unsigned long long* p, std::size_t n, unsigned long long v)
{
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
        p[i] = v;
    }
}

// ---- admission gate -------------------------------------------------------
// Per demand record: e = issue deferred past severe/shutdown windows; the
// gate is one server, a = max(e, g), g' = a + gap (gap = light_gap in light
// windows), i.e. the (max,+) map g -> max(g + gap, e + gap).

struct GArgs {
    const hbf_record32* rec;
    std::size_t n;
    std::uint64_t window_ps, windows, light_gap_ps;
    const std::uint8_t* level;     // [windows]
    const std::uint32_t* ok2;      // [windows + 1]: first window >= w with level < 2
};

// A block takes kGateTile records, kGatePer consecutive ones per thread.  The
// block first stages their issue times in LDS with coalesced loads, thread
// t's records in row t (rows padded by one word against bank conflicts);
// the admission times go back out the same way.
constexpr std::uint32_t kGatePer = 16;
constexpr std::uint32_t kGateTile = kThreads * kGatePer;
constexpr std::uint32_t kGateRow = kGatePer + 1;

__device__ __forceinline__ void stage_issue(const GArgs& g, std::size_t base, std::uint64_t* s)
{
    for (std::uint32_t k = threadIdx.x; k < kGateTile; k += kThreads) {
        const std::size_t i = base + k;
        s[(k / kGatePer) * kGateRow + k % kGatePer] = i < g.n ? g.rec[i].issue_ps : 0ull;
    }
    __syncthreads();
}

__device__ __forceinline__ void gate_record(const GArgs& g, std::uint64_t t, std::uint64_t& e,
                                            std::uint64_t& gap)
{
    const std::uint64_t w = t / g.window_ps;
    e = t;
    if (w < g.windows && g.level[w] >= 2) {
        e = static_cast<std::uint64_t>(g.ok2[w + 1]) * g.window_ps;
    }
    const std::uint64_t we = e / g.window_ps;
    gap = (we < g.windows && g.level[we] == 1) ? g.light_gap_ps : 0ull;
}

struct MaxPlus {
    std::uint64_t A, B;
};

__device__ __forceinline__ MaxPlus compose(MaxPlus f, MaxPlus s)
{
    // f first, then s
    const std::uint64_t b = f.B + s.A;
    return MaxPlus{f.A + s.A, b > s.B ? b : s.B};
}

// The map of a thread's `count` records (issue times in its LDS row).
__device__ MaxPlus thread_map(const GArgs& g, const std::uint64_t* row, std::uint32_t count)
{
    MaxPlus m{0, 0};
    for (std::uint32_t j = 0; j < count; ++j) {
        std::uint64_t e, gap;
        gate_record(g, row[j], e, gap);
        m = compose(m, MaxPlus{gap, e + gap});
    }
    return m;
}

// Records of this thread in the block's tile starting at `base`.
__device__ __forceinline__ std::uint32_t gate_count(const GArgs& g, std::size_t base)
{
    const std::size_t b = base + static_cast<std::size_t>(threadIdx.x) * kGatePer;
    return b < g.n ? static_cast<std::uint32_t>(std::min<std::size_t>(kGatePer, g.n - b)) : 0u;
}

// Inclusive scan of per-thread maps in thread order (Hillis-Steele).
__device__ MaxPlus block_scan(MaxPlus m, MaxPlus* sA)
{
    const int tid = threadIdx.x;
    sA[tid] = m;
    __syncthreads();
    for (int o = 1; o < kThreads; o <<= 1) {
        MaxPlus v = sA[tid];
        if (tid >= o) {
            v = compose(sA[tid - o], v);
        }
        __syncthreads();
        sA[tid] = v;
        __syncthreads();
    }
    return sA[tid];
}

__global__ __launch_bounds__(kThreads) void k_gate_summary(GArgs g, MaxPlus* tiles)
{
    __shared__ MaxPlus sA[kThreads];
    __shared__ std::uint64_t s_t[kThreads * kGateRow];
    const std::size_t base = static_cast<std::size_t>(blockIdx.x) * kGateTile;
    stage_issue(g, base, s_t);
    const std::uint32_t cnt = gate_count(g, base);
    const MaxPlus m =
        block_scan(thread_map(g, s_t + static_cast<std::size_t>(threadIdx.x) * kGateRow, cnt), sA);
    if (threadIdx.x == kThreads - 1) {
        tiles[blockIdx.x] = m;
    }
}

// One block: the gate value before every tile.
__global__ __launch_bounds__(kThreads) void k_gate_carry(const MaxPlus* tiles, std::size_t ntiles,
                                                         std::uint64_t* carry)
{
    __shared__ MaxPlus sA[kThreads];
    const std::size_t per = (ntiles + kThreads - 1) / kThreads;
    const std::size_t b = threadIdx.x * per, e = std::min(b + per, ntiles);
    MaxPlus m{0, 0};
    for (std::size_t t = b; t < e; ++t) {
        m = compose(m, tiles[t]);
    }
    const MaxPlus inc = block_scan(m, sA);
    __syncthreads();
    std::uint64_t gate = 0;
    if (threadIdx.x > 0) {
        const MaxPlus ex = sA[threadIdx.x - 1];
        gate = ex.A > ex.B ? ex.A : ex.B;  // map applied to g = 0
    }
    (void)inc;
    for (std::size_t t = b; t < e; ++t) {
        carry[t] = gate;
        const std::uint64_t x = gate + tiles[t].A;
        gate = x > tiles[t].B ? x : tiles[t].B;
    }
}

__global__ __launch_bounds__(kThreads) void k_gate_apply(GArgs g, const std::uint64_t* carry,
                                                         std::uint64_t* admit)
{
    __shared__ MaxPlus sA[kThreads];
    __shared__ std::uint64_t s_t[kThreads * kGateRow];
    const std::size_t base = static_cast<std::size_t>(blockIdx.x) * kGateTile;
    stage_issue(g, base, s_t);
    const std::uint32_t cnt = gate_count(g, base);
    std::uint64_t* row = s_t + static_cast<std::size_t>(threadIdx.x) * kGateRow;
    const MaxPlus mine = thread_map(g, row, cnt);
    block_scan(mine, sA);
    std::uint64_t gate = carry[blockIdx.x];
    if (threadIdx.x > 0) {
        const MaxPlus ex = sA[threadIdx.x - 1];
        const std::uint64_t x = gate + ex.A;
        gate = x > ex.B ? x : ex.B;
    }
    for (std::uint32_t j = 0; j < cnt; ++j) {  // admission times replace the issue times
        std::uint64_t ei, gap;
        gate_record(g, row[j], ei, gap);
        const std::uint64_t ai = ei > gate ? ei : gate;
        row[j] = ai;
        gate = ai + gap;
    }
    __syncthreads();
    for (std::uint32_t k = threadIdx.x; k < kGateTile; k += kThreads) {
        const std::size_t i = base + k;
        if (i < g.n) {
            admit[i] = s_t[(k / kGatePer) * kGateRow + k % kGatePer];
        }
    }
}

// Refresh j goes to j + #(demand admitted strictly before it).
__global__ void k_refresh_place(const hbf_record32* ref, std::size_t r,
                                const std::uint64_t* admit, std::size_t n, hbf_record32* merged)
{
    const std::size_t j = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
    if (j >= r) {
        return;
    }
    const std::uint64_t t = ref[j].issue_ps;
    std::size_t lo = 0, hi = n;
    while (lo < hi) {
        const std::size_t mid = (lo + hi) >> 1;
        if (admit[mid] < t) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    merged[j + lo] = ref[j];
}

// Demand i goes to i + #(refreshes admitted at or before it).
__global__ void k_merge_demand(const hbf_record32* rec, std::size_t n, const std::uint64_t* admit,
                               const std::uint64_t* ref_issue, std::size_t r,
                               hbf_record32* merged, std::uint64_t* pos)
{
    const std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
    if (i >= n) {
        return;
    }
    const std::uint64_t t = admit[i];
    std::size_t lo = 0, hi = r;
    while (lo < hi) {
        const std::size_t mid = (lo + hi) >> 1;
        if (ref_issue[mid] <= t) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    hbf_record32 v = rec[i];
    v.issue_ps = t;
    merged[i + lo] = v;
    pos[i] = i + lo;
}

struct Partial {
    unsigned long long deferred, modeled, lat_lo, lat_hi, lat_max;
};

__device__ __forceinline__ void add128(unsigned long long& lo, unsigned long long& hi,
                                       unsigned long long v)
{
    const unsigned long long s = lo + v;
    hi += s < lo ? 1ull : 0ull;
    lo = s;
}

// Demand completions back in input order, and the demand accounting.
__global__ __launch_bounds__(kThreads) void k_gather(const hbf_record32* rec, std::size_t n,
                                                     const std::uint64_t* admit,
                                                     const std::uint64_t* pos,
                                                     const std::uint64_t* mcomp,
                                                     const std::uint8_t* mstat,
                                                     std::uint64_t* completion, Partial* part)
{
    __shared__ Partial s[kThreads];
    Partial p{0, 0, 0, 0, 0};
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const std::uint64_t k = pos[i];
        const std::uint64_t c = mcomp[k];
        completion[i] = c;
        const std::uint64_t t = rec[i].issue_ps;
        p.deferred += admit[i] > t ? 1u : 0u;
        if ((mstat[k] & 3u) == 0) {
            const std::uint64_t lat = c - t;
            add128(p.lat_lo, p.lat_hi, lat);
            p.lat_max = lat > p.lat_max ? lat : p.lat_max;
            ++p.modeled;
        }
    }
    s[threadIdx.x] = p;
    __syncthreads();
    if (threadIdx.x == 0) {
        Partial t{0, 0, 0, 0, 0};
        for (int k = 0; k < kThreads; ++k) {
            t.deferred += s[k].deferred;
            t.modeled += s[k].modeled;
            t.lat_hi += s[k].lat_hi;
            add128(t.lat_lo, t.lat_hi, s[k].lat_lo);
            t.lat_max = s[k].lat_max > t.lat_max ? s[k].lat_max : t.lat_max;
        }
        part[blockIdx.x] = t;
    }
}

// ---------------------------------------------------------------------------

hipError_t halloc_bytes(void** p, std::size_t bytes)
{
    return hipMalloc(p, bytes == 0 ? 16 : bytes);
}

template <class T>
hipError_t halloc(T*& p, std::size_t count)
{
    return halloc_bytes(reinterpret_cast<void**>(&p), count * sizeof(T));
}

template <class T>
void hfree(T*& p)
{
    if (p != nullptr) {
        (void)hipFree(p);
        p = nullptr;
    }
}

// Tile edge in {16, 8, 4, 2, 1}: of those whose staged region fits in one
// workgroup and that divide div_x and div_y, the largest that still gives
// every CU a tile (256 tiles), else the smallest.
void choose_tile(std::uint32_t nx, std::uint32_t ny, std::uint32_t nz, std::uint32_t sweeps,
                 std::uint32_t div_x, std::uint32_t div_y, std::uint32_t& tx, std::uint32_t& ty)
{
    tx = ty = 0;
    for (std::uint32_t t = 16; t >= 1; t >>= 1) {
        const std::uint32_t r = t + 2 * sweeps;
        if (static_cast<std::uint64_t>(r) * r * nz <= kMaxRegion && div_x % t == 0 &&
            div_y % t == 0) {
            tx = ty = t;
            const std::uint64_t tiles = static_cast<std::uint64_t>((nx + t - 1) / t) *
                                        ((ny + t - 1) / t);
            if (tiles >= 256) {
                return;
            }
        }
    }
}

// Uncoupled steps: the largest square interior whose region fits a wide
// workgroup (when the device gives a workgroup that much LDS) and that still
// gives every CU a tile, if it re-reads fewer cells than choose_tile's tile;
// else choose_tile's.  Returns whether the tile is a wide one.
bool choose_step_tile(const hbfsim_amd_thermal_grid& g, std::size_t lds_per_block,
                      std::uint32_t& tx, std::uint32_t& ty)
{
    choose_tile(g.nx, g.ny, g.nz, g.sweeps, 16, 16, tx, ty);
    if (tx == 0) {
        return false;
    }
    for (std::uint32_t t = 64; t > tx; --t) {
        const std::uint64_t r = t + 2ull * g.sweeps;
        const std::uint64_t cells = r * r * g.nz;
        const std::uint64_t tiles =
            static_cast<std::uint64_t>((g.nx + t - 1) / t) * ((g.ny + t - 1) / t);
        if (cells <= kMaxWideRegion && 2 * (cells + 1) * sizeof(double) <= lds_per_block &&
            tiles >= 256 && t <= g.nx && t <= g.ny) {
            tx = ty = t;
            return true;
        }
    }
    return false;
}

std::uint64_t host_sat_add(std::uint64_t a, std::uint64_t b)
{
    return a > ~0ull - b ? ~0ull : a + b;
}

// cpu_service.cpp:221-255: control_sample, then apply_controls, at `now`
// with stack hotspot hs; returns the applied level.
std::uint32_t control_step(const hbfsim_amd_reliability_options& o, Ctl& c, std::uint64_t now,
                           double hs)
{
    const double thr[4] = {0.0, o.light_k, o.severe_k, o.shutdown_k};
    std::uint32_t desired = static_cast<std::uint32_t>(hs >= o.light_k) +
                            static_cast<std::uint32_t>(hs >= o.severe_k) +
                            static_cast<std::uint32_t>(hs >= o.shutdown_k);
    if (desired < c.applied && hs >= thr[c.applied] - o.hysteresis_k) {
        desired = c.applied;
    }
    if (o.policy != 0) {
        if (desired == c.applied) {
            c.pending = kNoPending;
        } else if (c.pending == kNoPending || c.pending != desired) {
            const std::uint64_t x = host_sat_add(now, o.action_delay_ps);
            const std::uint64_t y = host_sat_add(c.last_change, o.min_dwell_ps);
            c.pending = desired;
            c.pending_at = x > y ? x : y;
        }
    }
    if (c.pending != kNoPending && c.pending_at <= now) {
        c.applied = c.pending;
        c.last_change = now;
        c.pending = kNoPending;
    }
    return c.applied;
}

void host_retention_table(double ea, double tref, std::uint64_t window_ps, std::uint64_t* table)
{
    for (std::uint32_t b = 0; b < kAfBins; ++b) {
        const double t = kAfT0 + (static_cast<double>(b) + 0.5) / kAfStepsPerK;
        const double af = std::exp(ea / 8.62e-5 * (1.0 / tref - 1.0 / t));
        const double v = static_cast<double>(window_ps) * af;
        table[b] = v >= 1.8e19 ? ~0ull : static_cast<std::uint64_t>(std::llround(v));
    }
}

}  // namespace

struct thermal {
    hbfsim_amd_thermal_grid grid{};
    int device = 0;
    double* d_scratch = nullptr;   // second temperature buffer
    double* d_scratch2 = nullptr;  // third, made when an odd pass count first needs it
    std::uint64_t* d_wbase = nullptr;  // window counter of the coupled chain's graph
    hipStream_t cap = nullptr;         // stream the chain's graph is captured on
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipEvent_t cev[8] = {};        // coupled-run phase boundaries
    float last_ms = 0.0f;
    std::uint64_t last_launches = 0;  // kernel passes of the last thermal_step
    float phase_ms[5] = {};        // counts, thermal chain, admission, engine, gather
    std::size_t lds_per_block = 0;  // the device's LDS limit per workgroup
    bool wide_ready = false;        // the wide kernel may take that much LDS
    int cus = 0;                    // compute units
    // marching stencil (uncoupled steps on large grids), set up at the first step
    bool march_checked = false;
    bool march = false;
    MArgs m[2] = {};               // [0] one step per pass, [1] two (m_lds[1] == 0: none)
    std::uint32_t m_blocks[2] = {}, m_threads[2] = {};
    std::size_t m_lds[2] = {};
    // last coupled run
    std::uint64_t windows = 0;
    std::uint32_t ndie = 0;
    std::vector<double> hot;
    std::vector<std::uint8_t> level, refresh;
};

int thermal_create(const hbfsim_amd_thermal_grid& g, thermal** out)
{
    *out = nullptr;
    if (g.nx == 0 || g.ny == 0 || g.nz == 0 || g.sweeps == 0 || g.sweeps > 8 ||
        !(g.capacity_j_per_k > 0.0) || !(g.dt_s > 0.0) || !(g.gx_w_per_k >= 0.0) ||
        !(g.gy_w_per_k >= 0.0) || !(g.gz_w_per_k >= 0.0) || !(g.top_g_w_per_k >= 0.0) ||
        !std::isfinite(g.ambient_k)) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    int device = 0, lds_max = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, device) !=
            hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    const std::size_t lds_limit = lds_max > 0 ? static_cast<std::size_t>(lds_max) : 0;
    // steps take LDS tiles or, on large grids, the marching kernel
    std::uint32_t tx, ty;
    choose_tile(g.nx, g.ny, g.nz, g.sweeps, 16, 16, tx, ty);
    if (tx == 0 && march_lds(g, lds_limit) == 0) {
        return HBFSIM_UNSUPPORTED;
    }
    auto* th = new (std::nothrow) thermal;
    if (th == nullptr) {
        return HBFSIM_IO_ERROR;
    }
    th->grid = g;
    th->device = device;
    th->lds_per_block = lds_limit;
    hipError_t err = hipSuccess;
    if (err == hipSuccess)
        err = hipDeviceGetAttribute(&th->cus, hipDeviceAttributeMultiprocessorCount, th->device);
    if (err == hipSuccess)
        err = halloc(th->d_scratch, static_cast<std::size_t>(g.nx) * g.ny * g.nz);
    for (int i = 0; i < 2 && err == hipSuccess; ++i) {
        err = hipEventCreate(&th->ev[i]);
    }
    for (int i = 0; i < 8 && err == hipSuccess; ++i) {
        err = hipEventCreate(&th->cev[i]);
    }
    if (err != hipSuccess) {
        thermal_destroy(th);
        return HBFSIM_CUDA_ERROR;
    }
    *out = th;
    return HBFSIM_OK;
}

void thermal_destroy(thermal* th)
{
    if (th == nullptr) {
        return;
    }
    (void)hipSetDevice(th->device);
    (void)hipDeviceSynchronize();
    hfree(th->d_scratch);
    hfree(th->d_scratch2);
    hfree(th->d_wbase);
    if (th->cap != nullptr) {
        (void)hipStreamDestroy(th->cap);
    }
    for (auto& e : th->ev) {
        if (e != nullptr) {
            (void)hipEventDestroy(e);
        }
    }
    for (auto& e : th->cev) {
        if (e != nullptr) {
            (void)hipEventDestroy(e);
        }
    }
    delete th;
}

const hbfsim_amd_thermal_grid& thermal_get_grid(const thermal* th) { return th->grid; }

float thermal_last_step_ms(const thermal* th) { return th->last_ms; }

std::uint64_t thermal_last_launches(const thermal* th) { return th->last_launches; }

int coupled_last_ms(const thermal* th, float* ms, int max)
{
    const int k = max < 5 ? max : 5;
    for (int i = 0; i < k; ++i) {
        ms[i] = th->phase_ms[i];
    }
    return k;
}

namespace {

TArgs base_args(const hbfsim_amd_thermal_grid& g, std::uint32_t tx, std::uint32_t ty,
                std::uint32_t block = kTileBlock)
{
    TArgs a;
    std::memset(&a, 0, sizeof(a));
    a.nx = g.nx;
    a.ny = g.ny;
    a.nz = g.nz;
    a.sweeps = g.sweeps;
    a.tx = tx;
    a.ty = ty;
    a.rx = tx + 2 * g.sweeps;
    a.ry = ty + 2 * g.sweeps;
    a.tiles_x = (g.nx + tx - 1) / tx;
    a.cells = a.rx * a.ry * g.nz;
    a.block = block;
    a.step_x = block % a.rx;
    a.step_y = (block / a.rx) % a.ry;
    a.step_z = block / (a.rx * a.ry);
    a.cdt = g.capacity_j_per_k / g.dt_s;
    a.gx = g.gx_w_per_k;
    a.gy = g.gy_w_per_k;
    a.gz = g.gz_w_per_k;
    a.gb = g.top_g_w_per_k;
    a.tb = g.ambient_k;
    a.rw = a.rh = a.lpd = a.regions_x = a.D = 1;
    return a;
}

std::uint32_t tile_blocks(const TArgs& a)
{
    return a.tiles_x * ((a.ny + a.ty - 1) / a.ty);
}

// Segments are sized so that one round of resident workgroups covers the
// grid (or every strip is one segment when strips alone exceed a round).
// Rows are not balanced across strips: the strips of a segment walk the
// same rows at the same time, so HBM sees whole 16 KB rows rather than
// scattered pieces of them, which measured faster than equal row counts.

// One pass form (f steps per pass): its launch geometry.
hipError_t setup_march_form(thermal* th, int f)
{
    const auto& g = th->grid;
    const std::size_t lds = march_lds(g, th->lds_per_block, f);
    if (lds == 0) {
        return hipSuccess;
    }
    const void* fn = march_kernel(g.sweeps, f);
    const std::uint32_t levels = g.sweeps * static_cast<std::uint32_t>(f);
    const std::uint32_t W = kMarchLanes - 2 * levels;
    const std::uint32_t threads = kMarchLanes * g.nz;
    hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    int per_cu = 0;
    if (err == hipSuccess)
        err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, static_cast<int>(threads),
                                                           lds);
    if (err != hipSuccess || per_cu <= 0) {
        return err;
    }
    const std::uint32_t strips = (g.nx + W - 1) / W;
    const std::uint64_t round = static_cast<std::uint64_t>(per_cu) * th->cus;
    std::uint64_t segs = round / strips;
    const std::uint64_t max_segs = g.ny / (8ull * levels);  // segments of >= 8 L rows
    segs = std::max<std::uint64_t>(1, std::min(segs, max_segs));
    const std::uint32_t seg_len = static_cast<std::uint32_t>((g.ny + segs - 1) / segs);
    segs = (g.ny + seg_len - 1) / seg_len;
    MArgs& m = th->m[f - 1];
    m.nx = g.nx;
    m.ny = g.ny;
    m.nz = g.nz;
    m.strips = strips;
    m.seg_len = seg_len;
    m.total = static_cast<std::uint32_t>(strips * segs);
    m.per_xcd = (m.total + 7) / 8;
    m.cdt = g.capacity_j_per_k / g.dt_s;
    m.gx = g.gx_w_per_k;
    m.gy = g.gy_w_per_k;
    m.gz = g.gz_w_per_k;
    m.gb = g.top_g_w_per_k;
    m.tb = g.ambient_k;
    th->m_blocks[f - 1] = m.per_xcd * 8;
    th->m_threads[f - 1] = threads;
    th->m_lds[f - 1] = lds;
    return hipSuccess;
}

hipError_t setup_march(thermal* th)
{
    th->march_checked = true;
    if (th->cus <= 0) {
        return hipSuccess;
    }
    hipError_t err = setup_march_form(th, 1);
    if (err == hipSuccess && th->m_lds[0] != 0) {
        err = setup_march_form(th, 2);
        th->march = err == hipSuccess;
    }
    return err;
}

}  // namespace

int thermal_step(thermal* th, const double* d_power, double* d_temp, std::uint64_t steps,
                 void* stream_ptr)
{
    if (d_power == nullptr || d_temp == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (steps == 0) {
        return HBFSIM_OK;
    }
    if (hipSetDevice(th->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const auto& g = th->grid;
    if (!th->march_checked && setup_march(th) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    TArgs a{};
    std::size_t lds = 0;
    if (!th->march) {
        std::uint32_t tx, ty;
        const bool wide = choose_step_tile(g, th->lds_per_block, tx, ty);
        if (tx == 0) {
            return HBFSIM_UNSUPPORTED;  // no tile fits and the marching kernel does not apply
        }
        a = base_args(g, tx, ty, kTileBlock);
        a.power = d_power;
        lds = 2ull * (a.cells + 1) * sizeof(double);
        if (wide && !th->wide_ready) {
            if (hipFuncSetAttribute(
                    reinterpret_cast<const void*>(
                        k_thermal_window<false, kCellsPerThread, kTileBlock>),
                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
                hipSuccess) {
                return HBFSIM_CUDA_ERROR;
            }
            th->wide_ready = true;
        }
    }
    const std::size_t cells = static_cast<std::size_t>(g.nx) * g.ny * g.nz;
    // Passes: on the marching kernel pairs of steps in fused passes (the
    // power is the same in both) and the odd step in a single-step one.
    const std::uint64_t pairs = th->march && th->m_lds[1] != 0 ? steps / 2 : 0;
    const std::uint64_t launches = steps - pairs;
    // Each pass reads one buffer and writes another.  An even count
    // alternates d_temp and the scratch and ends in d_temp; an odd count of 3
    // or more goes d_temp -> scratch, then between the two scratch buffers,
    // and its last pass writes d_temp; a single pass leaves the result in the
    // scratch, copied back below.
    hipError_t err = hipSuccess;
    const bool three = (launches & 1) != 0 && launches >= 3;
    if (three && th->d_scratch2 == nullptr) {
        err = halloc(th->d_scratch2, cells);
        if (err != hipSuccess) {
            return HBFSIM_CUDA_ERROR;
        }
    }
    double* cur = d_temp;
    const auto target = [&](std::uint64_t i) {
        if (!three) {
            return cur == d_temp ? th->d_scratch : d_temp;
        }
        return i + 1 == launches ? d_temp : (cur == th->d_scratch ? th->d_scratch2 : th->d_scratch);
    };
    (void)hipEventRecord(th->ev[0], stream);
    for (std::uint64_t i = 0; i < launches && err == hipSuccess; ++i) {
        double* dst = target(i);
        if (th->march) {
            const int f = i < pairs ? 2 : 1;
            MArgs m = th->m[f - 1];
            m.power = d_power;
            err = march_launcher(g.sweeps, f)(m, th->m_blocks[f - 1], th->m_threads[f - 1],
                                              th->m_lds[f - 1], stream, cur, dst);
        } else {
            launch_window<false>(a, tile_blocks(a), lds, stream, cur, dst, 0ull);
        }
        cur = dst;
    }
    (void)hipEventRecord(th->ev[1], stream);
    if (err == hipSuccess) err = hipGetLastError();
    if (err == hipSuccess && cur != d_temp) {
        err = hipMemcpyAsync(d_temp, cur, cells * sizeof(double),
                             hipMemcpyDeviceToDevice, stream);
    }
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, th->ev[0], th->ev[1]) == hipSuccess) {
        th->last_ms = ms / static_cast<float>(steps);
    }
    th->last_launches = launches;
    return HBFSIM_OK;
}

// The coupled chain in captured chunks: kChainChunk windows (even, so each
// chunk ends on the buffers and ages it started from) whose kernels take
// their window index from a device counter, and a last node that advances
// it.  The graph holds the run's own buffers, so it is made per run; about
// 1.5 us of host time per window captured, against about 0.8 us saved per
// window replayed (a dependent kernel node starts in 1.7 us, a stream
// launch in 2.5 us).
constexpr std::uint64_t kChainChunk = 256;

struct ChainGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t stream = nullptr;  // where it was launched
    ~ChainGraph()
    {
        if (exec != nullptr) {
            (void)hipStreamSynchronize(stream);
            (void)hipGraphExecDestroy(exec);
        }
        if (graph != nullptr) {
            (void)hipGraphDestroy(graph);
        }
    }
};

hipError_t chain_graph(thermal* th, TArgs a, std::size_t lds, double* const buf[2],
                       std::uint64_t* d_age, std::uint32_t ndie, hipStream_t stream,
                       ChainGraph& cg)
{
    hipError_t err = hipSuccess;
    if (th->d_wbase == nullptr) {
        err = halloc(th->d_wbase, 1);
    }
    if (err == hipSuccess && th->cap == nullptr) {
        err = hipStreamCreateWithFlags(&th->cap, hipStreamNonBlocking);
    }
    if (err == hipSuccess) {
        err = hipStreamBeginCapture(th->cap, hipStreamCaptureModeThreadLocal);
    }
    if (err != hipSuccess) {
        return err;
    }
    a.wbase = th->d_wbase;
    for (std::uint64_t k = 0; k < kChainChunk; ++k) {
        a.age_in = d_age + (k & 1) * ndie;
        a.age_out = d_age + ((k + 1) & 1) * ndie;
        launch_window<true>(a, tile_blocks(a), lds, th->cap, buf[k & 1], buf[(k + 1) & 1], k);
    }
    hipLaunchKernelGGL(k_add_u64, dim3(1), dim3(64), 0, th->cap, th->d_wbase, kChainChunk);
    err = hipStreamEndCapture(th->cap, &cg.graph);
    if (err == hipSuccess) {
        err = hipGraphInstantiate(&cg.exec, cg.graph, nullptr, nullptr, 0);
    }
    cg.stream = stream;
    return err;
}

int coupled_run(engine* e, const engine_config& cfg, thermal* th,
                const hbfsim_amd_reliability_options& o, const hbf_record32* d_rec,
                std::size_t n, std::uint64_t* d_comp, double* d_temp, std::uint64_t* age,
                void* stream_ptr, hbfsim_amd_coupled_report* out, hbfsim_amd_report* erep)
{
    hbfsim_amd_coupled_report rep;
    std::memset(&rep, 0, sizeof(rep));
    if (out != nullptr) *out = rep;
    if (erep != nullptr) std::memset(erep, 0, sizeof(*erep));
    const auto& g = th->grid;
    const std::uint32_t cw = cfg.channels * cfg.ways;
    const std::uint32_t ndie = cw * cfg.dies;
    if (d_temp == nullptr || age == nullptr || (n != 0 && (d_rec == nullptr || d_comp == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (o.regions_x == 0 || o.regions_y == 0 || o.regions_x * o.regions_y != cw ||
        g.nx % o.regions_x != 0 || g.ny % o.regions_y != 0 || g.nz % cfg.dies != 0 ||
        o.window_ps == 0 || o.policy > 1) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (std::fabs(static_cast<double>(o.window_ps) * 1e-12 - g.dt_s) > 1e-9 * g.dt_s ||
        cfg.dies > 64 || ndie > kMaxDies || cfg.model != HBFSIM_AMD_MODEL_HBF) {
        return HBFSIM_UNSUPPORTED;
    }
    // The merged stream carries refresh records, which the engine times only
    // with at most one page register and without warp grouping: refused here,
    // before anything is allocated or written.
    if (cfg.grouping != 0 || cfg.slots == 2) {
        return HBFSIM_UNSUPPORTED;
    }
    const std::uint32_t rw = g.nx / o.regions_x, rh = g.ny / o.regions_y;
    std::uint32_t tx, ty;
    choose_tile(g.nx, g.ny, g.nz, g.sweeps, rw, rh, tx, ty);
    if (tx == 0 || g.sweeps > rw || g.sweeps > rh) {
        return HBFSIM_UNSUPPORTED;
    }
    if (hipSetDevice(th->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    std::uint64_t windows = 0;
    if (n != 0) {
        // demand records in issue order (the windows, admission gate and
        // merge follow it): any that goes back refuses the run before the
        // grid, the ages or the engine change
        std::uint32_t* d_back = nullptr;
        std::uint32_t back = 0;
        std::uint64_t last = 0;
        hipError_t e0 = halloc(d_back, 1);
        if (e0 == hipSuccess) e0 = hipMemcpyAsync(d_back, &back, 4, hipMemcpyHostToDevice, stream);
        if (e0 == hipSuccess && order_check(d_rec, false, n, d_back, stream_ptr) != HBFSIM_OK) {
            e0 = hipErrorLaunchFailure;
        }
        if (e0 == hipSuccess) e0 = hipMemcpyAsync(&back, d_back, 4, hipMemcpyDeviceToHost, stream);
        if (e0 == hipSuccess)
            e0 = hipMemcpyAsync(&last, &d_rec[n - 1].issue_ps, 8, hipMemcpyDeviceToHost, stream);
        if (e0 == hipSuccess) e0 = hipStreamSynchronize(stream);
        hfree(d_back);
        if (e0 != hipSuccess) {
            return HBFSIM_CUDA_ERROR;
        }
        if (back != 0) {
            return HBFSIM_INVALID_ARGUMENT;
        }
        windows = last / o.window_ps + 1;
    }
    rep.windows = windows;
    if (windows > (1ull << 26)) {
        return HBFSIM_UNSUPPORTED;
    }
    const std::size_t cells = static_cast<std::size_t>(g.nx) * g.ny * g.nz;

    std::uint32_t* d_counts = nullptr;
    unsigned long long* d_hot = nullptr;
    std::uint64_t* d_af = nullptr;
    std::uint64_t* d_age = nullptr;  // [2][ndie]
    std::uint8_t* d_level = nullptr;
    std::uint8_t* d_refresh = nullptr;
    std::uint32_t* d_ok2 = nullptr;
    MaxPlus* d_gtiles = nullptr;
    std::uint64_t* d_gcarry = nullptr;
    std::uint64_t* d_admit = nullptr;
    hbf_record32* d_ref = nullptr;
    std::uint64_t* d_ref_issue = nullptr;
    hbf_record32* d_merged = nullptr;
    std::uint64_t* d_pos = nullptr;
    std::uint64_t* d_mcomp = nullptr;
    std::uint8_t* d_mstat = nullptr;
    Partial* d_part = nullptr;
    auto release = [&]() {
        hfree(d_counts); hfree(d_hot); hfree(d_af); hfree(d_age);
        hfree(d_level); hfree(d_refresh); hfree(d_ok2); hfree(d_gtiles); hfree(d_gcarry);
        hfree(d_admit); hfree(d_ref); hfree(d_ref_issue); hfree(d_merged); hfree(d_pos);
        hfree(d_mcomp); hfree(d_mstat); hfree(d_part);
    };
    const std::size_t wd = static_cast<std::size_t>(windows) * ndie;
    hipError_t err = halloc(d_counts, wd + 2);
    if (err == hipSuccess) err = halloc(d_hot, wd + ndie);
    if (err == hipSuccess) err = halloc(d_af, kAfBins);
    if (err == hipSuccess) err = halloc(d_age, 2ull * ndie);
    if (err == hipSuccess) err = halloc(d_level, windows);
    if (err == hipSuccess) err = halloc(d_refresh, wd);
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    // 1. per-window, per-die access counts
    (void)hipEventRecord(th->cev[0], stream);
    const unsigned fill_blocks = static_cast<unsigned>(std::min<std::size_t>((wd + ndie + 255) / 256, 65536));
    hipLaunchKernelGGL(k_fill_u64, dim3(std::max(1u, fill_blocks)), dim3(256), 0, stream,
                       d_hot, wd + ndie, 0ull);
    int st = HBFSIM_OK;
    if (wd != 0) {
        hipLaunchKernelGGL(k_fill_u64, dim3(static_cast<unsigned>(std::min<std::size_t>((wd / 2 + 256) / 256, 65536))),
                           dim3(256), 0, stream, reinterpret_cast<unsigned long long*>(d_counts),
                           (wd * 4 + 7) / 8, 0ull);
        st = engine_window_counts(e, d_rec, n, o.window_ps, windows, d_counts, stream_ptr);
    }
    if (st != HBFSIM_OK) {
        release();
        return st;
    }
    // 2. thermal / retention / throttle chain
    (void)hipEventRecord(th->cev[1], stream);
    std::vector<std::uint64_t> table(kAfBins);
    host_retention_table(o.activation_energy_ev, o.reference_k, o.window_ps, table.data());
    err = hipMemcpyAsync(d_af, table.data(), kAfBins * 8, hipMemcpyHostToDevice, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(d_age, age, ndie * 8ull, hipMemcpyHostToDevice, stream);
    TArgs a = base_args(g, tx, ty, kTileBlock);
    a.coupled = 1;
    a.ndie = ndie;
    a.regions_x = o.regions_x;
    a.rw = rw;
    a.rh = rh;
    a.D = cfg.dies;
    a.lpd = g.nz / cfg.dies;
    a.static_w = o.static_power_w;
    const double cells_per_die = static_cast<double>(rw * rh * a.lpd);
    a.pa = (o.access_energy_j / g.dt_s) / cells_per_die;
    a.pr = (o.refresh_energy_j / g.dt_s) / cells_per_die;
    a.counts = d_counts;
    a.hot = d_hot;
    a.af = d_af;
    a.retention_ps = o.retention_ps;
    a.window_ps = o.window_ps;
    a.refresh = d_refresh;
    if (err == hipSuccess) {
        hipLaunchKernelGGL(k_die_hot, dim3(static_cast<unsigned>(std::min<std::size_t>((cells + 255) / 256, 4096))),
                           dim3(256), 0, stream, a, static_cast<const double*>(d_temp), d_hot);
    }
    const std::size_t lds = 2ull * (a.cells + 1) * sizeof(double);
    double* buf[2] = {d_temp, th->d_scratch};
    // Whole chunks of kChainChunk windows replay one captured graph (a
    // dependent kernel node starts sooner than a stream launch); the rest,
    // and any chunk whose capture fails, launch one by one.
    std::uint64_t w0 = 0;
    ChainGraph cg;
    if (err == hipSuccess && windows >= 2 * kChainChunk &&
        chain_graph(th, a, lds, buf, d_age, ndie, stream, cg) == hipSuccess) {
        hipLaunchKernelGGL(k_fill_u64, dim3(1), dim3(64), 0, stream,
                           reinterpret_cast<unsigned long long*>(th->d_wbase), std::size_t{1}, 0ull);
        for (; w0 + kChainChunk <= windows && err == hipSuccess; w0 += kChainChunk) {
            err = hipGraphLaunch(cg.exec, stream);
        }
    }
    for (std::uint64_t w = w0; w < windows && err == hipSuccess; ++w) {
        a.age_in = d_age + (w & 1) * ndie;
        a.age_out = d_age + ((w + 1) & 1) * ndie;
        launch_window<true>(a, tile_blocks(a), lds, stream, buf[w & 1], buf[(w + 1) & 1], w);
    }
    if (err == hipSuccess) err = hipGetLastError();
    (void)hipEventRecord(th->cev[2], stream);
    if (err == hipSuccess && (windows & 1)) {
        err = hipMemcpyAsync(d_temp, th->d_scratch, cells * sizeof(double),
                             hipMemcpyDeviceToDevice, stream);
    }
    th->hot.assign(wd + ndie, 0.0);
    th->level.assign(windows, 0);
    th->refresh.assign(wd, 0);
    if (err == hipSuccess)
        err = hipMemcpyAsync(age, d_age + (windows & 1) * ndie, ndie * 8ull, hipMemcpyDeviceToHost,
                             stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(th->hot.data(), d_hot, (wd + ndie) * 8, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess && wd)
        err = hipMemcpyAsync(th->refresh.data(), d_refresh, wd, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    th->windows = windows;
    th->ndie = ndie;
    // throttle levels from the stack hotspot of each window's start
    {
        Ctl c{0, kNoPending, 0, 0};
        for (std::uint64_t w = 0; w < windows; ++w) {
            const double* row = th->hot.data() + w * ndie;
            double hs = row[0];
            for (std::uint32_t d = 1; d < ndie; ++d) {
                hs = row[d] > hs ? row[d] : hs;
            }
            th->level[w] = static_cast<std::uint8_t>(control_step(o, c, w * o.window_ps, hs));
            rep.level_windows[th->level[w]] += 1;
        }
    }
    for (double v : th->hot) {
        rep.peak_k = v > rep.peak_k ? v : rep.peak_k;
    }

    // 3. admission, refresh records, merge
    std::vector<std::uint32_t> ok2(windows + 1), ok3(windows + 1);
    ok2[windows] = ok3[windows] = static_cast<std::uint32_t>(windows);
    for (std::uint64_t w = windows; w-- > 0;) {
        ok2[w] = th->level[w] < 2 ? static_cast<std::uint32_t>(w) : ok2[w + 1];
        ok3[w] = th->level[w] < 3 ? static_cast<std::uint32_t>(w) : ok3[w + 1];
    }
    std::vector<hbf_record32> refs;
    std::vector<std::uint64_t> ref_issue;
    {
        const std::uint32_t sizes[4] = {cfg.channels, cfg.ways, cfg.dies, cfg.planes};
        std::uint64_t div[4];
        std::uint64_t stride = 1;
        for (int i = 0; i < 4; ++i) {
            div[cfg.order[i]] = stride;
            stride *= sizes[cfg.order[i]];
        }
        const std::uint64_t pages = cfg.media_pages == ~0ull ? 0ull : cfg.media_pages;
        std::uint64_t rows = pages / stride;
        if (rows == 0) rows = 1;
        std::vector<std::uint64_t> ordinal(ndie, 0);
        for (std::uint64_t w = 0; w < windows; ++w) {
            for (std::uint32_t d = 0; d < ndie; ++d) {
                if (!th->refresh[w * ndie + d]) continue;
                const std::uint32_t q = d / cfg.dies, dd = d % cfg.dies;
                const std::uint64_t k = ordinal[d]++;
                const std::uint64_t coord[4] = {q / cfg.ways, q % cfg.ways, dd, k % cfg.planes};
                std::uint64_t page = ((k / cfg.planes) % rows) * stride;
                for (int ax = 0; ax < 4; ++ax) page += coord[ax] * div[ax];
                hbf_record32 r;
                r.addr = page;
                r.bytes = 2ull << cfg.page_shift;
                const std::uint64_t t = w * o.window_ps;
                r.issue_ps = th->level[w] >= 3 ? static_cast<std::uint64_t>(ok3[w + 1]) * o.window_ps : t;
                r.flags = 2u | 0x100u;
                refs.push_back(r);
                ref_issue.push_back(r.issue_ps);
            }
        }
    }
    const std::size_t nref = refs.size();
    rep.refreshes = nref;
    const std::size_t total = n + nref;
    const std::size_t gtiles = (n + kGateTile - 1) / kGateTile;
    err = halloc(d_ok2, windows + 1);
    if (err == hipSuccess) err = halloc(d_gtiles, gtiles);
    if (err == hipSuccess) err = halloc(d_gcarry, gtiles);
    if (err == hipSuccess) err = halloc(d_admit, n);
    if (err == hipSuccess) err = halloc(d_ref, nref);
    if (err == hipSuccess) err = halloc(d_ref_issue, nref);
    if (err == hipSuccess) err = halloc(d_merged, total);
    if (err == hipSuccess) err = halloc(d_pos, n);
    if (err == hipSuccess) err = halloc(d_mcomp, total);
    if (err == hipSuccess) err = halloc(d_mstat, total);
    const unsigned gblocks = static_cast<unsigned>(std::min<std::size_t>((n + kThreads - 1) / kThreads, 4096));
    if (err == hipSuccess) err = halloc(d_part, std::max(1u, gblocks));
    if (err == hipSuccess)
        err = hipMemcpyAsync(d_ok2, ok2.data(), ok2.size() * 4, hipMemcpyHostToDevice, stream);
    if (err == hipSuccess && windows)
        err = hipMemcpyAsync(d_level, th->level.data(), windows, hipMemcpyHostToDevice, stream);
    if (err == hipSuccess && nref)
        err = hipMemcpyAsync(d_ref, refs.data(), nref * sizeof(hbf_record32), hipMemcpyHostToDevice,
                             stream);
    if (err == hipSuccess && nref)
        err = hipMemcpyAsync(d_ref_issue, ref_issue.data(), nref * 8, hipMemcpyHostToDevice, stream);
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    (void)hipEventRecord(th->cev[3], stream);
    if (n != 0) {
        GArgs ga;
        ga.rec = d_rec;
        ga.n = n;
        ga.window_ps = o.window_ps;
        ga.windows = windows;
        ga.light_gap_ps = o.light_gap_ps;
        ga.level = d_level;
        ga.ok2 = d_ok2;
        hipLaunchKernelGGL(k_gate_summary, dim3(static_cast<unsigned>(gtiles)), dim3(kThreads), 0,
                           stream, ga, d_gtiles);
        hipLaunchKernelGGL(k_gate_carry, dim3(1), dim3(kThreads), 0, stream,
                           static_cast<const MaxPlus*>(d_gtiles), gtiles, d_gcarry);
        hipLaunchKernelGGL(k_gate_apply, dim3(static_cast<unsigned>(gtiles)), dim3(kThreads), 0,
                           stream, ga, static_cast<const std::uint64_t*>(d_gcarry), d_admit);
        hipLaunchKernelGGL(k_merge_demand, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                           0, stream, d_rec, n, static_cast<const std::uint64_t*>(d_admit),
                           static_cast<const std::uint64_t*>(d_ref_issue), nref, d_merged, d_pos);
    }
    if (nref != 0) {
        hipLaunchKernelGGL(k_refresh_place, dim3(static_cast<unsigned>((nref + 255) / 256)),
                           dim3(256), 0, stream, static_cast<const hbf_record32*>(d_ref), nref,
                           static_cast<const std::uint64_t*>(d_admit), n, d_merged);
    }
    err = hipGetLastError();
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    (void)hipEventRecord(th->cev[4], stream);
    // 4. the engine on the merged stream
    hbfsim_amd_report er;
    st = engine_run(e, d_merged, total, d_mcomp, d_mstat, 0, stream_ptr, &er, nref != 0);
    if (st != HBFSIM_OK) {
        release();
        return st;
    }
    rep.makespan_ps = er.makespan_ps;
    (void)hipEventRecord(th->cev[5], stream);
    if (n != 0) {
        hipLaunchKernelGGL(k_gather, dim3(gblocks), dim3(kThreads), 0, stream, d_rec, n,
                           static_cast<const std::uint64_t*>(d_admit),
                           static_cast<const std::uint64_t*>(d_pos),
                           static_cast<const std::uint64_t*>(d_mcomp),
                           static_cast<const std::uint8_t*>(d_mstat), d_comp, d_part);
        std::vector<Partial> parts(gblocks);
        (void)hipEventRecord(th->cev[6], stream);
        err = hipGetLastError();
        if (err == hipSuccess)
            err = hipMemcpyAsync(parts.data(), d_part, gblocks * sizeof(Partial),
                                 hipMemcpyDeviceToHost, stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
        if (err != hipSuccess) {
            release();
            return HBFSIM_CUDA_ERROR;
        }
        for (const Partial& p : parts) {
            rep.deferred += p.deferred;
            rep.demand_modeled += p.modeled;
            rep.latency_sum_hi += p.lat_hi;
            const std::uint64_t lo = rep.latency_sum_lo + p.lat_lo;
            rep.latency_sum_hi += lo < rep.latency_sum_lo ? 1u : 0u;
            rep.latency_sum_lo = lo;
            rep.latency_max_ps = std::max<std::uint64_t>(rep.latency_max_ps, p.lat_max);
        }
    }
    release();
    const int pairs[5][2] = {{0, 1}, {1, 2}, {3, 4}, {4, 5}, {5, 6}};
    for (int k = 0; k < 5; ++k) {
        float ms = 0.0f;
        th->phase_ms[k] = (n != 0 && hipEventElapsedTime(&ms, th->cev[pairs[k][0]],
                                                         th->cev[pairs[k][1]]) == hipSuccess)
                              ? ms
                              : 0.0f;
    }
    if (out != nullptr) *out = rep;
    if (erep != nullptr) *erep = er;
    return HBFSIM_OK;
}

int coupled_trace(const thermal* th, double* hot, std::size_t hot_count, std::uint8_t* level,
                  std::size_t level_count, std::uint8_t* refresh, std::size_t refresh_count,
                  std::uint64_t* windows, std::uint32_t* dies)
{
    if (windows != nullptr) *windows = th->windows;
    if (dies != nullptr) *dies = th->ndie;
    if ((hot != nullptr && hot_count < th->hot.size()) ||
        (level != nullptr && level_count < th->level.size()) ||
        (refresh != nullptr && refresh_count < th->refresh.size())) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (hot != nullptr && !th->hot.empty())
        std::memcpy(hot, th->hot.data(), th->hot.size() * sizeof(double));
    if (level != nullptr && !th->level.empty())
        std::memcpy(level, th->level.data(), th->level.size());
    if (refresh != nullptr && !th->refresh.empty())
        std::memcpy(refresh, th->refresh.data(), th->refresh.size());
    return HBFSIM_OK;
}

}  // namespace hbfamd
