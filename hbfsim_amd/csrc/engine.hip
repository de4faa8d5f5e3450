// engine.hip -- HBF per-access timing engine for gfx950 (MI355X).
//
// Replaces the reference's per-access device resolver and its single global
// busy-until tail (src/cuda_runtime/device/hbf_device.cu:765-959, 963-1344)
// with a batch pipeline over access records resident in HBM:
//
//   k_summary  one wave per tile of records: classify against the range
//              table (binary search, fences staged in LDS), stripe the media
//              page onto channel/way/die/plane, and fold every record into a
//              per-resource (max,+) summary of the tile.  Planes also carry
//              their page-register tag; a tile's first record on a plane has
//              its page-buffer hit resolved later, from the carry.
//   k_carry_*  a three-level scan over the tile summaries gives the exact
//              busy-until / tag state at the start of every tile (and the
//              final state, kept for the next run); one launch for runs of
//              at most 4,096 tiles, three for larger ones.
//   k_apply    re-reads each tile, replays it from its carry-in state and
//              writes completion times, status bytes and accounting.
//
// Per resource, busy' = max(busy, issue) + service.  The map
// b -> max(b + A, B) composes associatively,
//   (A1, B1) then (A2, B2) = (A1 + A2, max(B1 + A2, B2)),
// which is what lets a wave fold a group of same-resource records in
// log2(64) shuffle rounds and lets tiles be summarised independently.
//
// Within a step of 64 records the wave groups lanes by resource with 64-bit
// ballots (one per key bit), orders each group by lane, and scans it by
// pointer jumping.  No atomics touch timing state, so results are
// deterministic and bit-identical to the sequential CPU model.
#include <hip/hip_runtime.h>

#include "engine.hpp"
#include "thermal.hpp"

#include <algorithm>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

namespace hbfamd {
namespace {

constexpr int kWave = 64;
// Top level of the two-level range lookup (find_range), staged in LDS by
// every per-record kernel.  256 fences (2 KiB) rather than 512 let the
// summary pass hold 8 waves per CU instead of 7 at 512 planes.
constexpr std::uint32_t kMaxFences = 256;
// Planes: the summary pass keeps 33 B of state per plane in LDS, which at
// 4,096 planes (135 KB) still fits gfx950's 160 KB per workgroup.
constexpr std::uint32_t kMaxPlanes = 4096;
constexpr std::uint32_t kMaxChannels = 256;
constexpr std::uint32_t kClsModeled = 0;
constexpr std::uint32_t kClsBypass = 1;
constexpr std::uint32_t kClsUnsupported = 2;
constexpr std::uint32_t kClsInvalid = 3;  // lane beyond the tile
constexpr std::uint32_t kClsFollower = 5;  // shares an earlier record's request
constexpr std::uint8_t kStGrouped = 32;

struct alignas(16) PlaneSum {
    std::uint64_t fpage1;  // page + 1 of the tile's first record (0: none)
    std::uint64_t fissue;  // its issue time
    std::uint64_t rA, rB;  // (max,+) map of the records after the first
    std::uint64_t lpage1;  // page + 1 of the tile's last record
    std::uint32_t fcls;    // first record: bit 0 op, bit 1 programs
    std::uint32_t pad;
};
struct alignas(16) ChanSum {
    std::uint64_t A, B;
};
struct alignas(16) PlaneCarry {
    std::uint64_t busy, tag1;
};

struct DevReport {
    unsigned long long v[14];
};
static_assert(offsetof(hbfsim_amd_report, grouped) == sizeof(DevReport), "report layout");
enum {
    R_RECORDS, R_MODELED, R_BYPASS, R_UNSUPPORTED, R_READS, R_WRITES, R_HITS,
    R_PROGRAMS, R_HYBRID, R_MAKESPAN, R_LAT_LO, R_LAT_HI, R_LAT_MAX, R_SERVICE
};

// A split step's second run (its media page + 1, the lane it starts at and
// its range id), beside the step's descriptor, whose byte count then carries
// kSplitFlag.
struct alignas(16) SplitDesc {
    std::uint32_t page1b;
    std::uint32_t k;
    std::uint32_t ridb;
    std::uint32_t pad;
};
constexpr std::uint32_t kSplitFlag = 0x80000000u;

// Kernel arguments, passed by value.
struct KArgs {
    // ranges (structure of arrays, sorted by base)
    const std::uint64_t* r_base;
    const std::uint64_t* r_length;
    const std::uint64_t* r_file_offset;
    const std::uint32_t* r_meta;  // mode | permissions << 8
    const std::uint32_t* r_id;
    std::uint32_t r_count, r_stride, r_nfence;
    // geometry
    std::uint32_t Rp, Rc;           // planes, channels (resource counts)
    std::uint32_t W, D, P;
    std::uint32_t pbits, cbits;     // key widths for grouping
    std::uint32_t pow2;             // all axis sizes powers of two
    std::uint32_t axis_size[4];     // C W D P
    std::uint64_t axis_div[4];      // product of faster axis sizes
    std::uint32_t axis_shift[4];    // log2 of axis_div (pow2 only)
    std::uint32_t flat;             // one channel, one plane
    std::uint32_t page_shift;
    std::uint32_t slots;
    std::uint32_t contention;
    std::uint32_t transfer_page;
    std::uint32_t every_write;
    std::uint32_t hybrid;
    std::uint32_t hybrid_warmup;
    std::uint64_t hybrid_threshold;
    std::uint64_t read_ps, program_ps;
    std::uint64_t xfer_num, xfer_den, xfer_q;
    std::uint64_t xfer_pow2[33];    // transfer ps for 2^k bytes
    std::uint64_t media_pages;      // device capacity in pages
    std::uint32_t tile;
    std::uint32_t ext_hits;         // page-buffer hits given per record (K = 2)
    // the per-record passes match lane keys through per-wave LDS tables (one
    // 64-bit lane mask per plane and per channel) instead of one ballot per
    // key bit; set where the tables cost the passes no occupancy
    std::uint32_t match_lds;
    // the per-record passes' general steps look a media page's plane and
    // channel up in a per-wave LDS table of Rp entries (power-of-two axes:
    // both depend on the page modulo Rp only) instead of striping it; set
    // where the table costs the passes no occupancy
    std::uint32_t stripe_lds;
    // warp grouping: per record, how many records back its group's request
    // was made (0: its own request); null when the run does not group
    const std::uint8_t* lead;
    // hybrid runs: the range id of each linear step beside its descriptor
    // (the sampler's key needs it); null otherwise
    std::uint32_t* desc_rid;
    // split steps' second runs beside their descriptors (with the descriptors)
    SplitDesc* desc_split;
    // set to 1 by the summary pass when some record's issue time is below its
    // predecessor's; the carry chain then leaves the engine state untouched
    // and the engine times the stream again from a sorted copy (null: the
    // stream is known to be in issue order)
    std::uint32_t* disorder;
    // per tile, written by the summary pass of packed records: 1 when the
    // tile holds a split step (the apply pass then takes its split-capable
    // body), else 0; null when the run takes no linear batches
    std::uint8_t* tile_split;
};

// Record operations: 0 read, 1 write, and 2 refresh of media page `addr`
// (read out and programmed back), valid only with kMediaFlag.
constexpr std::uint32_t kOpRefresh = 2;
constexpr std::uint32_t kMediaFlag = 0x100;

struct Dec {
    std::uint32_t cls;
    std::uint32_t bits;    // bit 0 write or refresh, bit 1 programs, bit 2 refresh
    std::uint32_t plane, chan;
    std::uint32_t range_id;
    std::uint64_t page1;   // media page + 1
    std::uint64_t issue;
    std::uint64_t xfer;
    std::uint64_t xbytes;  // bytes the channel moves
};

__device__ __forceinline__ std::uint64_t shfl64(std::uint64_t v, int src)
{
    const int lo = __shfl(static_cast<int>(static_cast<std::uint32_t>(v)), src);
    const int hi = __shfl(static_cast<int>(static_cast<std::uint32_t>(v >> 32)), src);
    return (static_cast<std::uint64_t>(static_cast<std::uint32_t>(hi)) << 32) |
           static_cast<std::uint32_t>(lo);
}

__device__ __forceinline__ std::uint64_t umax64(std::uint64_t a, std::uint64_t b)
{
    return a > b ? a : b;
}

// Completion times are written once and not read again by the pass, so they
// are stored non-temporally: kept out of the caches, they leave the next
// step's records there (config 2: the apply pass 3% faster and the next
// summary pass 2-5%).
__device__ __forceinline__ void put_done(std::uint64_t* p, std::uint64_t v)
{
    __builtin_nontemporal_store(v, p);
}

__device__ __forceinline__ std::uint64_t lanemask_lt(int lane)
{
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// SplitMix64 finaliser, the reference's fast_hash (hbf_device.cuh:729-736).
__device__ __forceinline__ std::uint64_t mix64(std::uint64_t v)
{
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

// Lanes whose key equals this lane's key, among `active`: one ballot per key
// bit.  Every lane of the wave must call it (uniform control flow).
__device__ __forceinline__ std::uint64_t match_key(std::uint32_t key, std::uint32_t bits,
                                                   std::uint64_t active)
{
    std::uint64_t m = active;
    for (std::uint32_t b = 0; b < bits; ++b) {
        const bool bit = (key >> b) & 1u;
        const std::uint64_t ones = __ballot(bit);
        m &= bit ? ones : ~ones;
    }
    return m;
}

// Inclusive scan of (A, B) maps over each lane group, in lane order, by
// pointer jumping along `pred` (the previous lane of the same group, or -1).
__device__ __forceinline__ void group_scan(std::uint64_t& A, std::uint64_t& B, int pred,
                                           int lane)
{
    int ptr = pred;
    for (int s = 0; s < 6; ++s) {
        if (__ballot(ptr >= 0) == 0) {
            break;
        }
        const int src = ptr < 0 ? lane : ptr;
        const std::uint64_t pA = shfl64(A, src);
        const std::uint64_t pB = shfl64(B, src);
        const int pp = __shfl(ptr, src);
        if (ptr >= 0) {
            B = umax64(pB + A, B);
            A = pA + A;
            ptr = pp;
        }
    }
}

// Two independent group scans of 32-bit (A, B) maps, interleaved: pointer
// jumping along pred1 and pred2 (previous lane of the same group, or -1).
__device__ __forceinline__ void group_scan32x2(std::uint32_t& A1, std::uint32_t& B1, int pred1,
                                               std::uint32_t& A2, std::uint32_t& B2, int pred2,
                                               int lane)
{
    int p1 = pred1, p2 = pred2;
    for (int s = 0; s < 6; ++s) {
        if (__ballot(p1 >= 0 || p2 >= 0) == 0) {
            break;
        }
        const int s1 = p1 < 0 ? lane : p1;
        const int s2 = p2 < 0 ? lane : p2;
        const std::uint32_t a1 = static_cast<std::uint32_t>(__shfl(static_cast<int>(A1), s1));
        const std::uint32_t b1 = static_cast<std::uint32_t>(__shfl(static_cast<int>(B1), s1));
        const int q1 = __shfl(p1, s1);
        const std::uint32_t a2 = static_cast<std::uint32_t>(__shfl(static_cast<int>(A2), s2));
        const std::uint32_t b2 = static_cast<std::uint32_t>(__shfl(static_cast<int>(B2), s2));
        const int q2 = __shfl(p2, s2);
        if (p1 >= 0) {
            const std::uint32_t nb = b1 + A1;
            B1 = nb > B1 ? nb : B1;
            A1 = a1 + A1;
            p1 = q1;
        }
        if (p2 >= 0) {
            const std::uint32_t nb = b2 + A2;
            B2 = nb > B2 ? nb : B2;
            A2 = a2 + A2;
            p2 = q2;
        }
    }
}

// Whole-wave inclusive scan of (A, B) maps in lane order, for steps where
// every active lane belongs to one group (inactive lanes hold the identity
// (0, 0)).  DPP row shifts build 16-lane scans, then row broadcasts join the
// rows; no LDS traffic.  Controls are the GFX9 encodings gfx950 keeps:
// row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int Ctrl, int RowMask>
__device__ __forceinline__ std::uint64_t dpp64(std::uint64_t v)
{
    const int lo = __builtin_amdgcn_update_dpp(
        0, static_cast<int>(static_cast<std::uint32_t>(v)), Ctrl, RowMask, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(
        0, static_cast<int>(static_cast<std::uint32_t>(v >> 32)), Ctrl, RowMask, 0xF, false);
    return (static_cast<std::uint64_t>(static_cast<std::uint32_t>(hi)) << 32) |
           static_cast<std::uint32_t>(lo);
}

template <int Ctrl, int RowMask>
__device__ __forceinline__ void dpp_scan_step(std::uint64_t& A, std::uint64_t& B)
{
    const std::uint64_t pA = dpp64<Ctrl, RowMask>(A);
    const std::uint64_t pB = dpp64<Ctrl, RowMask>(B);
    B = umax64(pB + A, B);
    A = pA + A;
}

__device__ __forceinline__ void wave_scan(std::uint64_t& A, std::uint64_t& B)
{
    dpp_scan_step<0x111, 0xF>(A, B);
    dpp_scan_step<0x112, 0xF>(A, B);
    dpp_scan_step<0x114, 0xF>(A, B);
    dpp_scan_step<0x118, 0xF>(A, B);
    dpp_scan_step<0x142, 0xA>(A, B);
    dpp_scan_step<0x143, 0xC>(A, B);
}

template <int Ctrl, int RowMask>
__device__ __forceinline__ void dpp_scan_step32(std::uint32_t& A, std::uint32_t& B)
{
    const std::uint32_t pA = static_cast<std::uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(A), Ctrl, RowMask, 0xF, false));
    const std::uint32_t pB = static_cast<std::uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(B), Ctrl, RowMask, 0xF, false));
    const std::uint32_t nb = pB + A;
    B = nb > B ? nb : B;
    A = pA + A;
}

// Two independent whole-wave scans in 32 bits, interleaved for ILP.
__device__ __forceinline__ void wave_scan32x2(std::uint32_t& A1, std::uint32_t& B1,
                                              std::uint32_t& A2, std::uint32_t& B2)
{
    dpp_scan_step32<0x111, 0xF>(A1, B1);
    dpp_scan_step32<0x111, 0xF>(A2, B2);
    dpp_scan_step32<0x112, 0xF>(A1, B1);
    dpp_scan_step32<0x112, 0xF>(A2, B2);
    dpp_scan_step32<0x114, 0xF>(A1, B1);
    dpp_scan_step32<0x114, 0xF>(A2, B2);
    dpp_scan_step32<0x118, 0xF>(A1, B1);
    dpp_scan_step32<0x118, 0xF>(A2, B2);
    dpp_scan_step32<0x142, 0xA>(A1, B1);
    dpp_scan_step32<0x142, 0xA>(A2, B2);
    dpp_scan_step32<0x143, 0xC>(A1, B1);
    dpp_scan_step32<0x143, 0xC>(A2, B2);
}

// Inclusive prefix maximum across the wave (DPP; lanes without a source take
// 0, the identity for unsigned max).
template <int Ctrl, int RowMask>
__device__ __forceinline__ std::uint32_t dpp32(std::uint32_t v)
{
    return static_cast<std::uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), Ctrl, RowMask, 0xF, false));
}

__device__ __forceinline__ std::uint32_t wave_prefix_max32(std::uint32_t v)
{
    std::uint32_t t;
    t = dpp32<0x111, 0xF>(v); v = v > t ? v : t;
    t = dpp32<0x112, 0xF>(v); v = v > t ? v : t;
    t = dpp32<0x114, 0xF>(v); v = v > t ? v : t;
    t = dpp32<0x118, 0xF>(v); v = v > t ? v : t;
    t = dpp32<0x142, 0xA>(v); v = v > t ? v : t;
    t = dpp32<0x143, 0xC>(v); v = v > t ? v : t;
    return v;
}

__device__ __forceinline__ std::uint64_t wave_prefix_max64(std::uint64_t v)
{
    std::uint64_t t;
    t = dpp64<0x111, 0xF>(v); v = umax64(v, t);
    t = dpp64<0x112, 0xF>(v); v = umax64(v, t);
    t = dpp64<0x114, 0xF>(v); v = umax64(v, t);
    t = dpp64<0x118, 0xF>(v); v = umax64(v, t);
    t = dpp64<0x142, 0xA>(v); v = umax64(v, t);
    t = dpp64<0x143, 0xC>(v); v = umax64(v, t);
    return v;
}

__device__ __forceinline__ std::uint64_t readlane64(std::uint64_t v, int lane)
{
    const std::uint32_t lo = static_cast<std::uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<std::uint32_t>(v)), lane));
    const std::uint32_t hi = static_cast<std::uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<std::uint32_t>(v >> 32)), lane));
    return (static_cast<std::uint64_t>(hi) << 32) | lo;
}

// find_range_index (hbf_device.cuh:826-841): upper_bound(base) - 1 over the
// sorted range table.  The top level runs over every `stride`-th base,
// staged in LDS; the bottom level over at most `stride` bases in memory.
__device__ __forceinline__ std::uint32_t find_range(const KArgs& a, const std::uint64_t* fence,
                                                    std::uint64_t addr)
{
    std::uint32_t lo = 0, hi = a.r_nfence;
    while (lo < hi) {
        const std::uint32_t mid = (lo + hi) >> 1;
        if (fence[mid] <= addr) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    if (lo == 0) {
        return a.r_count;
    }
    const std::uint32_t start = (lo - 1) * a.r_stride;
    std::uint32_t end = start + a.r_stride;
    end = end < a.r_count ? end : a.r_count;
    std::uint32_t l2 = start + 1, h2 = end;
    while (l2 < h2) {
        const std::uint32_t mid = (l2 + h2) >> 1;
        if (a.r_base[mid] <= addr) {
            l2 = mid + 1;
        } else {
            h2 = mid;
        }
    }
    return l2 - 1;
}

// range_overlaps (hbf_device.cuh:873-884)
__device__ __forceinline__ bool overlaps(std::uint64_t base, std::uint64_t length,
                                         std::uint64_t addr, std::uint64_t bytes)
{
    if (bytes == 0 || length == 0 || base > ~0ull - length || addr > ~0ull - bytes) {
        return false;
    }
    return addr < base + length && base < addr + bytes;
}

__device__ __forceinline__ std::uint64_t xfer_ps(const KArgs& a, std::uint64_t bytes)
{
    if ((bytes & (bytes - 1)) == 0 && bytes != 0 && bytes <= (1ull << 32)) {
        return a.xfer_pow2[63 - __clzll(bytes)];
    }
    return a.xfer_q * ((bytes * a.xfer_num + a.xfer_den - 1) / a.xfer_den);
}

// The same with the power-of-two table in LDS, for per-lane byte counts: a
// lane-indexed read of the kernel arguments would be a vector memory load,
// and the record pipeline keeps those out of the step loop.
__device__ __forceinline__ std::uint64_t xfer_ps_lds(const KArgs& a, const std::uint64_t* xp,
                                                     std::uint64_t bytes)
{
    if ((bytes & (bytes - 1)) == 0 && bytes != 0 && bytes <= (1ull << 32)) {
        return xp[63 - __clzll(bytes)];
    }
    return a.xfer_q * ((bytes * a.xfer_num + a.xfer_den - 1) / a.xfer_den);
}

// Copies the power-of-two transfer table into LDS (`xp`, 33 entries).
__device__ __forceinline__ void load_xfer_table(const KArgs& a, std::uint64_t* xp, int lane)
{
    if (lane < 33) {
        xp[lane] = a.xfer_pow2[lane];
    }
}

// The same in two halves, so that later loads can be issued in between.
__device__ __forceinline__ std::uint64_t fetch_xfer(const KArgs& a, int lane)
{
    return lane < 33 ? a.xfer_pow2[lane] : 0ull;
}

__device__ __forceinline__ void store_xfer(std::uint64_t* xp, std::uint64_t v, int lane)
{
    if (lane < 33) {
        xp[lane] = v;
    }
}

// Waits for every outstanding vector memory operation (s_waitcnt vmcnt(0)).
// Called where a step has just made its own per-lane loads, so that none of
// them is still outstanding when the next step starts: the record pipeline's
// group in flight is then waited on only when the wave needs it.
__device__ __forceinline__ void wait_vector_loads()
{
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt 0, expcnt 7, lgkmcnt 15: vmcnt only
}

// Range last found by this lane.  Ranges are disjoint, so an address inside
// the cached range is inside no other one and the search can be skipped.
struct RangeCache {
    std::uint64_t base;
    std::uint64_t end;
    std::uint64_t file_offset;
    std::uint32_t meta;
    std::uint32_t id;
};

__device__ __forceinline__ RangeCache empty_cache()
{
    RangeCache c;
    c.base = 1;
    c.end = 0;
    c.file_offset = 0;
    c.meta = 0;
    c.id = 0;
    return c;
}

__device__ __forceinline__ void load_record(const hbf_record32* rec, std::size_t i, uint4& x,
                                            uint4& y)
{
    const uint4* p = reinterpret_cast<const uint4*>(rec + i);
    x = p[0];
    y = p[1];
}

// Records reach a wave in groups of kPipe steps: while the wave works through
// one group (held in registers), the next group's loads are in flight, so
// each wave keeps kPipe * 2 KiB of reads outstanding for kPipe steps of
// work.  (A load queue rotated one step at a time would wait on the newest
// load at every step, since the rotation copies it.)  A step's 2 KiB arrive
// coalesced, 16 B per lane: half A holds records 0..31 and half B records
// 32..63, lane l holding word pair l & 1 of record l >> 1 (even lanes address
// and bytes, odd lanes issue time and operation).  Loading record-per-lane
// instead (32 B stride) caps the read rate at ~4.8 TB/s; the coalesced form
// streams at ~6.3 TB/s.  Within the current group the next step is always
// slot 0: taking a step shifts the group down by one slot, register moves
// with constant indices that wait on nothing in flight (a selection by step
// index would put the group in scratch memory).
constexpr int kPipe = 4;
// The summary pass of 32-byte records, whose occupancy its per-plane LDS
// state limits (not its registers), keeps twice as many steps in flight per
// wave.
constexpr int kSumPipe = 8;
// Packed records in the summary pass: four waves per SIMD with three steps in
// flight each.  Measured against three waves with eight steps: general
// streams +8% per step (k_summary 4.15 -> 3.57 ms at 2^28 records) and the
// paged-KV step +15%, the TinyLlama step 2% slower; the LDS-bound variant
// (kDeep) keeps 2 * kSumPipe at two waves.  A run whose tiles all fit in one
// round of three-wave slots (kFewTiles) leaves SIMDs without a fourth wave
// anyway: it keeps three waves with kSumPipe steps in flight (kFew).
constexpr int kPackedSumPipe = 3;
constexpr std::size_t kFewTiles = 3 * 4 * 256;  // waves per SIMD x SIMDs per CU x CUs
// Linear-step detection on streams that show none: after kLinGiveUp steps in
// a row fail it, a wave probes only every kLinProbe-th step until one
// passes (every step is exact on the general path too; random streams stop
// paying for the check).
constexpr std::uint32_t kLinGiveUp = 8;
constexpr std::size_t kLinProbe = 32;

// A step in the registers of one lane: the coalesced halves of 32-byte
// records, or one packed 16-byte record.
struct Step32 {
    uint4 A, B;
};
struct Step16 {
    uint4 R;
};

// Records are read once per pass and streamed, so their loads are
// non-temporal: they then leave the caches to what the passes read again (the
// tile summaries, descriptors and carries).  Config 2: the step 6% faster.
__device__ __forceinline__ uint4 load_stream(const uint4* p)
{
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

template <int D>
struct RecordPipeT {
    using Step = Step32;
    uint4 ca[D], cb[D];  // the group being worked through
    uint4 na[D], nb[D];  // the next group, in flight

    __device__ __forceinline__ void issue(const void* rec, std::size_t g, std::size_t end,
                                          int lane)
    {
        const uint4* p = reinterpret_cast<const uint4*>(rec);
        if (g + static_cast<std::size_t>(D) * kWave <= end) {
            // the whole group lies inside the tile (every group but a tile's
            // last): plain loads, no per-load bounds or zero fill
            const uint4* q = p + 2 * g + static_cast<std::size_t>(lane);
#pragma unroll
            for (int j = 0; j < D; ++j) {
                na[j] = load_stream(q + static_cast<std::size_t>(2 * j) * kWave);
                nb[j] = load_stream(q + static_cast<std::size_t>(2 * j + 1) * kWave);
            }
            return;
        }
        const std::size_t words = 2 * end;  // 16-byte words in the tile's records
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const std::size_t w = 2 * (g + static_cast<std::size_t>(j) * kWave) + lane;
            na[j] = make_uint4(0, 0, 0, 0);
            nb[j] = na[j];
            if (w < words) {
                na[j] = p[w];
            }
            if (w + kWave < words) {
                nb[j] = p[w + kWave];
            }
        }
    }
    // Makes the group in flight current (waiting for it).
    __device__ __forceinline__ void promote()
    {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            ca[j] = na[j];
            cb[j] = nb[j];
        }
    }
    // Makes the group in flight current and issues the one after it.
    __device__ __forceinline__ void advance(const void* rec, std::size_t next, std::size_t end,
                                            int lane)
    {
        promote();
        if (next < end) {
            issue(rec, next, end, lane);
        }
    }
    // The current group's next step, in the coalesced halves.
    __device__ __forceinline__ void take(Step32& st)
    {
        st.A = ca[0];
        st.B = cb[0];
#pragma unroll
        for (int j = 0; j + 1 < D; ++j) {
            ca[j] = ca[j + 1];
            cb[j] = cb[j + 1];
        }
    }
};

// Packed records (hbf_record16, 16 B): word 0 holds the address (bits 0-47)
// and byte count (bits 48-63), word 1 the issue time (bits 0-55) and the
// operation (bits 56-63).  A step is 1 KiB and lane r loads record r whole,
// so no transpose is needed, and a group holds one register quad per step.
template <int D>
struct PackedPipeT {
    using Step = Step16;
    uint4 c[D];   // the group being worked through
    uint4 nx[D];  // the next group, in flight

    __device__ __forceinline__ void issue(const void* rec, std::size_t g, std::size_t end,
                                          int lane)
    {
        const uint4* p = reinterpret_cast<const uint4*>(rec);
        if (g + static_cast<std::size_t>(D) * kWave <= end) {
            const uint4* q = p + g + static_cast<std::size_t>(lane);
#pragma unroll
            for (int j = 0; j < D; ++j) {
                nx[j] = load_stream(q + static_cast<std::size_t>(j) * kWave);
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const std::size_t i = g + static_cast<std::size_t>(j) * kWave + lane;
            nx[j] = make_uint4(0, 0, 0, 0);
            if (i < end) {
                nx[j] = p[i];
            }
        }
    }
    __device__ __forceinline__ void promote()
    {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            c[j] = nx[j];
        }
    }
    __device__ __forceinline__ void advance(const void* rec, std::size_t next, std::size_t end,
                                            int lane)
    {
        promote();
        if (next < end) {
            issue(rec, next, end, lane);
        }
    }
    __device__ __forceinline__ void take(Step16& st)
    {
        st.R = c[0];
#pragma unroll
        for (int j = 0; j + 1 < D; ++j) {
            c[j] = c[j + 1];
        }
    }
};

// A packed record in the two word quads the decoder takes (x: address,
// bytes; y: issue time, operation).
__device__ __forceinline__ void unpack16(const uint4& r, uint4& x, uint4& y)
{
    x = make_uint4(r.x, r.y & 0xffffu, r.y >> 16, 0u);
    y = make_uint4(r.z, r.w & 0xffffffu, r.w >> 24, 0u);
}

using RecordPipe = RecordPipeT<kPipe>;

// Record-per-lane form of a step (lane r gets record r's two word pairs).
__device__ __forceinline__ void to_records(const uint4& A, const uint4& B, int lane, uint4& x,
                                           uint4& y)
{
    const int sx = ((2 * lane) & 63) << 2;  // bpermute byte addresses
    const int sy = ((2 * lane + 1) & 63) << 2;
    const bool lo = lane < 32;
    const auto pick = [&](std::uint32_t a, std::uint32_t b, int src) {
        const std::uint32_t ta =
            static_cast<std::uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(a)));
        const std::uint32_t tb =
            static_cast<std::uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(b)));
        return lo ? ta : tb;
    };
    x = make_uint4(pick(A.x, B.x, sx), pick(A.y, B.y, sx), pick(A.z, B.z, sx),
                   pick(A.w, B.w, sx));
    y = make_uint4(pick(A.x, B.x, sy), pick(A.y, B.y, sy), pick(A.z, B.z, sy), 0);
}

__device__ __forceinline__ void step_records(const Step32& st, int lane, uint4& x, uint4& y)
{
    to_records(st.A, st.B, lane, x, y);
}

__device__ __forceinline__ void step_records(const Step16& st, int, uint4& x, uint4& y)
{
    unpack16(st.R, x, y);
}

// Channel and global plane id of a media page (the profile's allocation
// scheme, fastest axis first).
__device__ __forceinline__ void stripe(const KArgs& a, std::uint64_t page, Dec& d)
{
    if (a.flat) {
        return;
    }
    std::uint32_t c[4];
    if (a.pow2) {
#pragma unroll
        for (int ax = 0; ax < 4; ++ax) {
            c[ax] = static_cast<std::uint32_t>((page >> a.axis_shift[ax]) &
                                               (a.axis_size[ax] - 1));
        }
    } else {
#pragma unroll
        for (int ax = 0; ax < 4; ++ax) {
            c[ax] = static_cast<std::uint32_t>((page / a.axis_div[ax]) % a.axis_size[ax]);
        }
    }
    d.chan = c[0];
    d.plane = ((c[0] * a.W + c[1]) * a.D + c[2]) * a.P + c[3];
}

// A wave's stripe table: entry r = plane | channel << 20 of media page r,
// r < Rp.  With power-of-two axes every axis digit is a bit field of the
// page's low log2(Rp) bits, so page p stripes as p mod Rp does.
__device__ __forceinline__ void fill_stripe_table(const KArgs& a, std::uint32_t* stab, int lane)
{
    for (std::uint32_t r = static_cast<std::uint32_t>(lane); r < a.Rp; r += kWave) {
        Dec d;
        d.plane = 0;
        d.chan = 0;
        stripe(a, r, d);
        stab[r] = d.plane | (d.chan << 20);
    }
}

// The operation a decoded record carries (hybrid sampler key).
__device__ __forceinline__ std::uint32_t dec_op(std::uint32_t bits)
{
    return (bits & 4u) ? kOpRefresh : (bits & 1u);
}

// Classification in the resolver's order (hbf_device.cu:1081-1165) followed
// by striping of the media page.  Refresh records are recognised only in
// the kRefresh instantiation (streams the thermal-coupled run merged them
// into); the other streams keep the branch out of the hot loop.  `stab`:
// the wave's stripe table (fill_stripe_table), when the run keeps one.
template <bool kRefresh, bool kUniform = false>
__device__ __forceinline__ Dec decode(const KArgs& a, const std::uint64_t* fence, RangeCache& rc,
                                      const uint4& x, const uint4& y, std::uint64_t base_ps,
                                      const std::uint32_t* stab = nullptr)
{
    const std::uint64_t addr = x.x | (static_cast<std::uint64_t>(x.y) << 32);
    const std::uint64_t bytes = x.z | (static_cast<std::uint64_t>(x.w) << 32);
    const std::uint64_t issue_rel = y.x | (static_cast<std::uint64_t>(y.y) << 32);
    const std::uint32_t op = y.z & 0xffu;
    Dec d;
    d.issue = base_ps + issue_rel;
    d.bits = op & 1u;
    d.plane = 0;
    d.chan = 0;
    d.range_id = 0;
    d.page1 = 0;
    d.xfer = 0;
    d.xbytes = 0;
    if (kRefresh && op == kOpRefresh && (y.z & kMediaFlag) != 0) {
        if (bytes == 0 || bytes > 0xffffffffull || addr >= a.media_pages) {
            d.cls = kClsUnsupported;
            return d;
        }
        d.cls = kClsModeled;
        d.bits = 7u;
        d.page1 = addr + 1;
        d.xbytes = bytes;
        stripe(a, addr, d);
        return d;
    }
    if (!(addr >= rc.base && addr < rc.end)) {
        std::uint32_t idx = find_range(a, fence, addr);
        if (kUniform) {
            // wave-uniform record: keep the range in scalar registers
            idx = static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(idx)));
        }
        if (idx == a.r_count || addr < a.r_base[idx] ||
            addr - a.r_base[idx] >= a.r_length[idx]) {
            const std::uint32_t succ = idx == a.r_count ? 0u : idx + 1u;
            if (bytes > 0xffffffffull ||
                (succ < a.r_count && overlaps(a.r_base[succ], a.r_length[succ], addr, bytes))) {
                d.cls = kClsUnsupported;
            } else {
                d.cls = kClsBypass;
            }
            return d;
        }
        rc.base = a.r_base[idx];
        rc.end = rc.base + a.r_length[idx];
        rc.file_offset = a.r_file_offset[idx];
        rc.meta = a.r_meta[idx];
        rc.id = a.r_id[idx];
        if (!kUniform) {
            wait_vector_loads();
        }
    }
    const std::uint32_t mode = rc.meta & 0xffu;
    const std::uint32_t perms = rc.meta >> 8;
    const std::uint64_t page_mask = (1ull << a.page_shift) - 1;
    // access_supported (hbf_device.cuh:843-860); the range's own bounds and
    // page size are validated at registration.
    if (bytes == 0 || bytes > 0xffffffffull || op > 1 || (mode != 1 && mode != 2) ||
        bytes > ~0ull - addr || addr + bytes > rc.end || (perms & (1u << op)) == 0) {
        d.cls = kClsUnsupported;
        return d;
    }
    const std::uint64_t off = addr - rc.base;
    if ((off >> a.page_shift) != ((off + bytes - 1) >> a.page_shift)) {
        d.cls = kClsUnsupported;
        return d;
    }
    if ((off & ~page_mask) > ~0ull - rc.file_offset) {
        d.cls = kClsUnsupported;
        return d;
    }
    d.cls = kClsModeled;
    d.range_id = rc.id;
    const std::uint64_t media = rc.file_offset + off;
    const std::uint64_t page = media >> a.page_shift;
    d.page1 = page + 1;
    const std::uint64_t page_bytes = 1ull << a.page_shift;
    if (op == 1 && (a.every_write || (media & page_mask) + bytes == page_bytes)) {
        d.bits |= 2u;
    }
    d.xbytes = a.transfer_page ? page_bytes : bytes;
    // (striping written out here rather than through stripe(): the helper
    // costs the summary kernel a quarter of its speed)
    if (!a.flat && stab != nullptr) {
        // plane | channel << 20 of the page modulo Rp (a power of two)
        const std::uint32_t e = stab[static_cast<std::uint32_t>(page) & (a.Rp - 1)];
        d.chan = e >> 20;
        d.plane = e & 0xfffffu;
    } else if (!a.flat) {
        std::uint32_t c[4];
        if (a.pow2) {
#pragma unroll
            for (int ax = 0; ax < 4; ++ax) {
                c[ax] = static_cast<std::uint32_t>((page >> a.axis_shift[ax]) &
                                                   (a.axis_size[ax] - 1));
            }
        } else {
#pragma unroll
            for (int ax = 0; ax < 4; ++ax) {
                c[ax] = static_cast<std::uint32_t>((page / a.axis_div[ax]) % a.axis_size[ax]);
            }
        }
        d.chan = c[0];
        d.plane = ((c[0] * a.W + c[1]) * a.D + c[2]) * a.P + c[3];
    }
    return d;
}

__device__ __forceinline__ Dec invalid_dec()
{
    Dec d;
    d.cls = kClsInvalid;
    d.bits = 0;
    d.plane = d.chan = d.range_id = 0;
    d.page1 = d.issue = d.xfer = d.xbytes = 0;
    return d;
}

// Transfer time of every lane's access.  When all modeled lanes move the same
// byte count (the usual case) it is computed once, in scalar registers.
__device__ __forceinline__ std::uint64_t lane_xfer(const KArgs& a, const std::uint64_t* xp,
                                                   const Dec& d, bool m, std::uint64_t active)
{
    const int first = __ffsll(static_cast<long long>(active)) - 1;
    const std::uint32_t lo = static_cast<std::uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<std::uint32_t>(d.xbytes)), first));
    const std::uint32_t hi = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(
        static_cast<int>(static_cast<std::uint32_t>(d.xbytes >> 32)), first));
    const std::uint64_t xb0 = (static_cast<std::uint64_t>(hi) << 32) | lo;
    if (__ballot(m && d.xbytes != xb0) == 0) {
        return xfer_ps(a, xb0);
    }
    return m ? xfer_ps_lds(a, xp, d.xbytes) : 0ull;
}

// Time origin for 32-bit scans: the first active lane's issue time.  The
// narrow path is taken only when, for every modeled lane, issue - origin is
// in [0, 2^30) and both services are below 2^24, so every partial sum of a
// step fits 32 bits.  (0, 0) in relative form stands for (0, origin), which
// acts as the identity on every state reachable in the step.
struct Narrow {
    std::uint64_t origin;
    bool ok;
};

__device__ __forceinline__ Narrow narrow_check(const Dec& d, bool m, std::uint64_t active,
                                               std::uint64_t svc1, std::uint64_t svc2)
{
    const int first = __ffsll(static_cast<long long>(active)) - 1;
    Narrow n;
    n.origin = shfl64(d.issue, first);
    const bool bad = m && (d.issue < n.origin || d.issue - n.origin >= (1ull << 30) ||
                           svc1 >= (1ull << 24) || svc2 >= (1ull << 24));
    n.ok = __ballot(bad) == 0;
    return n;
}

// A sequential run step: all 64 lanes are modeled reads of one media page,
// with the same byte count, in non-decreasing issue order (weight and KV
// streaming produce these).  With at least one page register, lanes 1..63
// hit the page their predecessor just read (plane map (0, issue_i)), and with
// a constant transfer x the channel maps fold to one prefix maximum:
//   lane i's channel map = (x (i + 1), x (i + 1) + max_{k<=i} (issue_k - x k)).
// Wave-uniform.
__device__ __forceinline__ bool run_step(const KArgs& a, const Dec& d, std::uint64_t active,
                                         int lane)
{
    if (active != ~0ull || a.slots == 0) {
        return false;
    }
    const std::uint32_t page0 = static_cast<std::uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<std::uint32_t>(d.page1)), 0));
    const std::uint64_t bytes0 = readlane64(d.xbytes, 0);
    const std::uint64_t prev = shfl64(d.issue, lane == 0 ? 0 : lane - 1);
    const bool bad = static_cast<std::uint32_t>(d.page1) != page0 || (d.bits & 1u) != 0 ||
                     d.xbytes != bytes0 || d.issue < prev;
    return __ballot(bad) == 0;
}

// W_i = max_{k<=i} (issue_k + x (63 - k)) for a run step, so that the channel
// completion of lane i is max(cursor + x (i + 1), W_i - x (62 - i)).  Runs in
// 32 bits relative to lane 0's issue when the step's span allows.
__device__ __forceinline__ std::uint64_t run_channel_max(const Dec& d, std::uint64_t x, int lane)
{
    const std::uint64_t w = d.issue + x * static_cast<std::uint64_t>(63 - lane);
    const std::uint64_t i0 = readlane64(d.issue, 0);
    const std::uint64_t i63 = readlane64(d.issue, 63);
    if (i63 - i0 + 64 * x < (1ull << 31) && x < (1ull << 24)) {
        return i0 + wave_prefix_max32(static_cast<std::uint32_t>(w - i0));
    }
    return wave_prefix_max64(w);
}

__device__ __forceinline__ std::uint32_t rfl32(std::uint32_t v)
{
    return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// A linear step: 64 reads addr_0 + k * bytes_0 with one issue time, inside
// one page of one range (weight streaming issues whole page-halves in one
// slot).  Such a step touches one plane and one channel; lanes 1..63 hit the
// page lane 0 opened, so its effect has a closed form given lane 0's record.
// linear_detect checks a step in scalar registers against the wave-uniform
// range cache (the full decode runs only when the cache misses) and returns
// the step's media page + 1, issue time and byte count.  Anything else (and
// any step with fewer than 64 records) takes the general paths.
__device__ __forceinline__ std::uint32_t rl32(std::uint32_t v, int k)
{
    return static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), k));
}

// The range and page checks of a step whose 64 records already follow
// record 0 (xu: its address and bytes, yu: its issue time and operation).
template <bool kRefresh>
__device__ __forceinline__ bool linear_tail(const KArgs& a, const std::uint64_t* fence,
                                            RangeCache& rcu, const uint4& xu, const uint4& yu,
                                            std::uint64_t base_ps, std::uint32_t& page1,
                                            std::uint64_t& issue0, std::uint32_t& bytes0);

template <bool kRefresh>
__device__ __forceinline__ bool linear_detect(const KArgs& a, const std::uint64_t* fence,
                                              RangeCache& rcu, const Step32& st,
                                              std::uint64_t base_ps, bool full, int lane,
                                              std::uint32_t& page1, std::uint64_t& issue0,
                                              std::uint32_t& bytes0)
{
    if (!full) {
        return false;
    }
    const uint4& A = st.A;
    const uint4& B = st.B;
    // record 0: address and bytes in lane 0, issue and operation in lane 1
    const uint4 xu = make_uint4(rfl32(A.x), rfl32(A.y), rfl32(A.z), rfl32(A.w));
    const uint4 yu = make_uint4(rl32(A.x, 1), rl32(A.y, 1), rl32(A.z, 1), 0);
    if ((yu.z & 0xffu) != 0 || xu.w != 0 || xu.z == 0) {
        return false;  // reads of 1 .. 2^32 - 1 bytes only
    }
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    // lane l checks word pair l & 1 of records l >> 1 (half A) and 32 + (l >> 1) (half B)
    const std::uint64_t ea = a0 + static_cast<std::uint64_t>(lane >> 1) * xu.z;
    const std::uint64_t eb = ea + 32ull * xu.z;
    const std::uint64_t wa = A.x | (static_cast<std::uint64_t>(A.y) << 32);
    const std::uint64_t wb = B.x | (static_cast<std::uint64_t>(B.y) << 32);
    const bool odd = (lane & 1) != 0;
    const bool ok_even = wa == ea && A.z == xu.z && A.w == 0 && wb == eb && B.z == xu.z &&
                         B.w == 0;
    const bool ok_odd = A.x == yu.x && A.y == yu.y && A.z == yu.z && B.x == yu.x &&
                        B.y == yu.y && B.z == yu.z;
    if (__ballot(odd ? !ok_odd : !ok_even) != 0) {
        return false;
    }
    return linear_tail<kRefresh>(a, fence, rcu, xu, yu, base_ps, page1, issue0, bytes0);
}

// A packed step: lane l checks its own record against record 0.
template <bool kRefresh>
__device__ __forceinline__ bool linear_detect(const KArgs& a, const std::uint64_t* fence,
                                              RangeCache& rcu, const Step16& st,
                                              std::uint64_t base_ps, bool full, int lane,
                                              std::uint32_t& page1, std::uint64_t& issue0,
                                              std::uint32_t& bytes0)
{
    if (!full) {
        return false;
    }
    const uint4& R = st.R;
    const uint4 r0 = make_uint4(rfl32(R.x), rfl32(R.y), rfl32(R.z), rfl32(R.w));
    uint4 xu, yu;
    unpack16(r0, xu, yu);
    if (yu.z != 0 || xu.z == 0) {
        return false;  // reads of at least one byte only
    }
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    const std::uint64_t mine = a0 + static_cast<std::uint64_t>(lane) * xu.z;
    const bool ok = R.x == static_cast<std::uint32_t>(mine) &&
                    (R.y & 0xffffu) == (mine >> 32) && (R.y >> 16) == xu.z && R.z == r0.z &&
                    R.w == r0.w;
    if (__ballot(!ok) != 0) {
        return false;
    }
    return linear_tail<kRefresh>(a, fence, rcu, xu, yu, base_ps, page1, issue0, bytes0);
}

template <bool kRefresh>
__device__ __forceinline__ bool linear_tail(const KArgs& a, const std::uint64_t* fence,
                                            RangeCache& rcu, const uint4& xu, const uint4& yu,
                                            std::uint64_t base_ps, std::uint32_t& page1,
                                            std::uint64_t& issue0, std::uint32_t& bytes0)
{
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    if (!(a0 >= rcu.base && a0 < rcu.end)) {
        // refill the cache through the full classification
        const Dec d = decode<kRefresh, true>(a, fence, rcu, xu, yu, base_ps);
        if (d.cls != kClsModeled) {
            return false;
        }
    }
    // every record inside the cached range, which admits reads, and in one
    // page whose media offset does not wrap (access_supported,
    // hbf_device.cuh:843-860, for all 64 records at once)
    const std::uint32_t mode = rcu.meta & 0xffu;
    const std::uint64_t span = 64ull * xu.z;
    if ((mode != 1 && mode != 2) || (rcu.meta & (1u << 8)) == 0 || span > rcu.end - a0) {
        return false;
    }
    const std::uint64_t off0 = a0 - rcu.base;
    const std::uint64_t page_mask = (1ull << a.page_shift) - 1;
    if ((off0 >> a.page_shift) != ((off0 + span - 1) >> a.page_shift) ||
        (off0 & ~page_mask) > ~0ull - rcu.file_offset) {
        return false;
    }
    page1 = static_cast<std::uint32_t>(((rcu.file_offset + off0) >> a.page_shift) + 1);
    issue0 = base_ps + (yu.x | (static_cast<std::uint64_t>(yu.y) << 32));
    bytes0 = xu.z;
    return true;
}

// A linear step (k = 0: one run of 64) or a split step (two linear runs,
// lanes 0 .. k-1 and k .. 63, with one issue time and byte count).
struct LinStep {
    std::uint32_t page1, page1b, k, bytes, rid, ridb;
    std::uint64_t issue;
};

// Packed steps: a step whose records all share record 0's byte count, issue
// time and read operation, and whose addresses continue record 0's (one run,
// split where a page boundary falls inside it) or continue record 0's up to
// a lane k and lane k's after it (two spans joined).  Each run must lie in
// one page of a range that admits reads (access_supported,
// hbf_device.cuh:843-860, for the run's records at once); a run whose first
// address lies outside the wave-uniform range cache refills it through the
// full classification (one call site for both runs).
template <bool kRefresh>
__device__ __forceinline__ bool linear_detect_split(const KArgs& a, const std::uint64_t* fence,
                                                    RangeCache& rcu, const Step16& st,
                                                    std::uint64_t base_ps, bool full, int lane,
                                                    LinStep& ls)
{
    if (!full) {
        return false;
    }
    const uint4& R = st.R;
    const uint4 r0 = make_uint4(rfl32(R.x), rfl32(R.y), rfl32(R.z), rfl32(R.w));
    uint4 xu, yu;
    unpack16(r0, xu, yu);
    if (yu.z != 0 || xu.z == 0) {
        return false;  // reads of at least one byte only
    }
    const std::uint32_t b0 = xu.z;
    if (__ballot((R.y >> 16) != b0 || R.z != r0.z || R.w != r0.w) != 0) {
        return false;
    }
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    const std::uint64_t addr = R.x | (static_cast<std::uint64_t>(R.y & 0xffffu) << 32);
    const std::uint64_t breaks = __ballot(addr != a0 + static_cast<std::uint64_t>(lane) * b0);
    std::uint32_t k = 0;  // the split lane (0: none)
    std::uint64_t a1 = 0;
    if (breaks != 0) {
        k = static_cast<std::uint32_t>(__ffsll(static_cast<long long>(breaks)) - 1);
        a1 = readlane64(addr, static_cast<int>(k));
        const std::uint64_t own =
            a1 + static_cast<std::uint64_t>(lane - static_cast<int>(k)) * b0;
        if (__ballot(lane >= static_cast<int>(k) && addr != own) != 0) {
            return false;
        }
    }
    ls.issue = base_ps + (yu.x | (static_cast<std::uint64_t>(yu.y) << 32));
    ls.bytes = b0;
    ls.page1b = 0;
    ls.ridb = 0;
    const std::uint64_t page_mask = (1ull << a.page_shift) - 1;
    std::uint64_t at = a0;
    std::uint32_t cnt = k != 0 ? k : static_cast<std::uint32_t>(kWave);
    for (int part = 0; part < 2; ++part) {
        if (!(at >= rcu.base && at < rcu.end)) {
            const uint4 xa = make_uint4(static_cast<std::uint32_t>(at),
                                        static_cast<std::uint32_t>(at >> 32), b0, 0u);
            const Dec d = decode<kRefresh, true>(a, fence, rcu, xa, yu, base_ps);
            if (d.cls != kClsModeled) {
                return false;
            }
        }
        const std::uint32_t mode = rcu.meta & 0xffu;
        if ((mode != 1 && mode != 2) || (rcu.meta & (1u << 8)) == 0) {
            return false;
        }
        const std::uint64_t off = at - rcu.base;
        std::uint64_t span = static_cast<std::uint64_t>(cnt) * b0;
        if ((off >> a.page_shift) != ((off + span - 1) >> a.page_shift)) {
            // one run crossing a page boundary: split it there when the
            // boundary falls between two records
            const std::uint64_t room = (off | page_mask) + 1 - off;
            if (part != 0 || k != 0 || room % b0 != 0) {
                return false;
            }
            k = static_cast<std::uint32_t>(room / b0);
            a1 = a0 + room;
            cnt = k;
            span = room;
        }
        if (span > rcu.end - at || (off & ~page_mask) > ~0ull - rcu.file_offset) {
            return false;
        }
        const std::uint32_t page1 =
            static_cast<std::uint32_t>(((rcu.file_offset + off) >> a.page_shift) + 1);
        if (part == 0) {
            ls.page1 = page1;
            ls.rid = rcu.id;
            if (k == 0) {
                break;  // a whole linear step
            }
        } else {
            ls.page1b = page1;
            ls.ridb = rcu.id;
        }
        at = a1;
        cnt = static_cast<std::uint32_t>(kWave) - k;
    }
    ls.k = k;
    return true;
}

// The step detection of a record form: packed steps may be split (kSplit);
// otherwise, and for 32-byte records, steps are whole linear steps or none.
template <bool kRefresh, bool kSplit>
__device__ __forceinline__ bool detect_step(const KArgs& a, const std::uint64_t* fence,
                                            RangeCache& rcu, const Step16& st,
                                            std::uint64_t base_ps, bool full, int lane,
                                            LinStep& ls)
{
    if constexpr (kSplit) {
        return linear_detect_split<kRefresh>(a, fence, rcu, st, base_ps, full, lane, ls);
    }
    ls.k = 0;
    ls.page1b = 0;
    ls.ridb = 0;
    const bool lin = linear_detect<kRefresh>(a, fence, rcu, st, base_ps, full, lane, ls.page1,
                                             ls.issue, ls.bytes);
    ls.rid = rcu.id;
    return lin;
}

template <bool kRefresh, bool kSplit>
__device__ __forceinline__ bool detect_step(const KArgs& a, const std::uint64_t* fence,
                                            RangeCache& rcu, const Step32& st,
                                            std::uint64_t base_ps, bool full, int lane,
                                            LinStep& ls)
{
    ls.k = 0;
    ls.page1b = 0;
    ls.ridb = 0;
    const bool lin = linear_detect<kRefresh>(a, fence, rcu, st, base_ps, full, lane, ls.page1,
                                             ls.issue, ls.bytes);
    ls.rid = rcu.id;
    return lin;
}

// A linear group: D consecutive linear steps continuing one another
// (record r of the group at address a0 + r * bytes0), each step with its own
// issue time, all inside the cached range.  Checked at once on the group's
// registers: lane l looks at word pair l & 1 of records 64 j + 32 h + (l >> 1)
// for every step j and half h.  The step values live one step per lane
// (lane j < D: step j), not in D wave-uniform registers each: per-step
// scalar arrays would hold about 3 D scalar registers across the group's
// checks, more than the wave has beside the kernel's own, and the overflow
// goes to VGPR lanes one write and one read at a time.
template <int D>
struct GroupLin {
    std::uint32_t page1;  // lane j < D: step j's media page + 1
    std::uint64_t issue;  // lane j < D: step j's issue time
    std::uint32_t bytes;
};

template <bool kRefresh, int D>
__device__ __forceinline__ bool group_tail(const KArgs& a, const std::uint64_t* fence,
                                           RangeCache& rcu, std::uint64_t base_ps,
                                           const uint4& xu, std::uint32_t op0, std::uint32_t vlo,
                                           std::uint32_t vhi, int lane, GroupLin<D>& gl);

template <bool kRefresh, int D>
__device__ __forceinline__ bool group_linear(const KArgs& a, const std::uint64_t* fence,
                                             RangeCache& rcu, const RecordPipeT<D>& pipe,
                                             std::uint64_t base_ps, int lane, GroupLin<D>& gl)
{
    const uint4 xu = make_uint4(rfl32(pipe.ca[0].x), rfl32(pipe.ca[0].y), rfl32(pipe.ca[0].z),
                                rfl32(pipe.ca[0].w));
    const std::uint32_t op0 = rl32(pipe.ca[0].z, 1);
    if ((op0 & 0xffu) != 0 || xu.w != 0 || xu.z == 0) {
        return false;  // reads of 1 .. 2^32 - 1 bytes only
    }
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    const std::uint64_t b0 = xu.z;
    const std::uint64_t half = 32ull * b0;  // bytes between the two halves of a step
    const std::uint64_t mine = a0 + static_cast<std::uint64_t>(lane >> 1) * b0;
    const bool odd = (lane & 1) != 0;
    std::uint32_t vlo = 0, vhi = 0;  // lane j < D: step j's issue time
    bool ok = true;
#pragma unroll
    for (int j = 0; j < D; ++j) {
        const std::uint32_t ilo = rl32(pipe.ca[j].x, 1);
        const std::uint32_t ihi = rl32(pipe.ca[j].y, 1);
        vlo = lane == j ? ilo : vlo;
        vhi = lane == j ? ihi : vhi;
        const uint4& A = pipe.ca[j];
        const uint4& B = pipe.cb[j];
        const std::uint64_t ea = mine + static_cast<std::uint64_t>(2 * j) * half;
        const std::uint64_t eb = ea + half;
        const std::uint64_t wa = A.x | (static_cast<std::uint64_t>(A.y) << 32);
        const std::uint64_t wb = B.x | (static_cast<std::uint64_t>(B.y) << 32);
        const bool ev = wa == ea && A.z == xu.z && A.w == 0 && wb == eb && B.z == xu.z &&
                        B.w == 0;
        const bool od = A.x == ilo && A.y == ihi && A.z == op0 && B.x == ilo && B.y == ihi &&
                        B.z == op0;
        ok = ok && (odd ? od : ev);
    }
    if (__ballot(!ok) != 0) {
        return false;
    }
    return group_tail<kRefresh, D>(a, fence, rcu, base_ps, xu, op0, vlo, vhi, lane, gl);
}

// A packed group: lane l checks its own record of every step.
template <bool kRefresh, int D>
__device__ __forceinline__ bool group_linear(const KArgs& a, const std::uint64_t* fence,
                                             RangeCache& rcu, const PackedPipeT<D>& pipe,
                                             std::uint64_t base_ps, int lane, GroupLin<D>& gl)
{
    const uint4 r0 = make_uint4(rfl32(pipe.c[0].x), rfl32(pipe.c[0].y), rfl32(pipe.c[0].z),
                                rfl32(pipe.c[0].w));
    uint4 xu, yu;
    unpack16(r0, xu, yu);
    if (yu.z != 0 || xu.z == 0) {
        return false;  // reads of at least one byte only
    }
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    const std::uint64_t b0 = xu.z;
    const std::uint64_t mine = a0 + static_cast<std::uint64_t>(lane) * b0;
    std::uint32_t vlo = 0, vhi = 0;  // lane j < D: step j's issue time
    bool ok = true;
#pragma unroll
    for (int j = 0; j < D; ++j) {
        const uint4& R = pipe.c[j];
        const std::uint32_t w = rfl32(R.w);  // record 0 of step j: issue high, operation
        const std::uint32_t ilo = rfl32(R.z);
        vlo = lane == j ? ilo : vlo;
        vhi = lane == j ? (w & 0xffffffu) : vhi;
        const std::uint64_t e = mine + static_cast<std::uint64_t>(j) * 64ull * b0;
        ok = ok && (w >> 24) == 0 && R.x == static_cast<std::uint32_t>(e) &&
             (R.y & 0xffffu) == (e >> 32) && (R.y >> 16) == b0 && R.z == ilo && R.w == w;
    }
    if (__ballot(!ok) != 0) {
        return false;
    }
    return group_tail<kRefresh, D>(a, fence, rcu, base_ps, xu, 0u, vlo, vhi, lane, gl);
}

// The range and page checks of a group whose records already continue one
// another from record 0 (xu: its address and bytes; op0: its operation;
// vlo, vhi: lane j < D holds step j's issue time), and the group's step
// values, lane j checking and holding step j.
template <bool kRefresh, int D>
__device__ __forceinline__ bool group_tail(const KArgs& a, const std::uint64_t* fence,
                                           RangeCache& rcu, std::uint64_t base_ps,
                                           const uint4& xu, std::uint32_t op0, std::uint32_t vlo,
                                           std::uint32_t vhi, int lane, GroupLin<D>& gl)
{
    static_assert(D <= kWave, "one lane per step");
    const std::uint64_t a0 = xu.x | (static_cast<std::uint64_t>(xu.y) << 32);
    const std::uint64_t b0 = xu.z;
    if (!(a0 >= rcu.base && a0 < rcu.end)) {
        const uint4 yu = make_uint4(rl32(vlo, 0), rl32(vhi, 0), op0, 0);
        const Dec d = decode<kRefresh, true>(a, fence, rcu, xu, yu, base_ps);
        if (d.cls != kClsModeled) {
            return false;
        }
    }
    const std::uint32_t mode = rcu.meta & 0xffu;
    const std::uint64_t step = 64ull * b0;
    const std::uint64_t span = D * step;
    if ((mode != 1 && mode != 2) || (rcu.meta & (1u << 8)) == 0 || span > rcu.end - a0) {
        return false;
    }
    const std::uint64_t page_mask = (1ull << a.page_shift) - 1;
    const std::uint64_t off = a0 - rcu.base + static_cast<std::uint64_t>(lane) * step;
    // a step crossing a page, or a page whose file offset overflows
    const bool bad = lane < D && ((off >> a.page_shift) != ((off + step - 1) >> a.page_shift) ||
                                  (off & ~page_mask) > ~0ull - rcu.file_offset);
    if (__ballot(bad) != 0) {
        return false;
    }
    gl.page1 = static_cast<std::uint32_t>(((rcu.file_offset + off) >> a.page_shift) + 1);
    gl.issue = base_ps + (vlo | (static_cast<std::uint64_t>(vhi) << 32));
    gl.bytes = xu.z;
    return true;
}

// What the summary pass learned about a step, for the apply pass: a linear
// step's media page + 1, byte count and issue time (bytes == 0: any other
// step).  Indexed by record index / 64.
struct alignas(16) StepDesc {
    std::uint32_t page1;
    std::uint32_t bytes;
    std::uint64_t issue;
};

// Linear steps waiting to be folded, as runs: lane r (r < n) holds run r --
// m consecutive records of one step, issued together and reading one page
// (its media page + 1, byte count and issue time), starting at lane lo of
// that step.  A whole linear step is one run (m = 64, lo = 0); a split step
// (two linear runs, split at lane k: a page boundary inside the step, or two
// spans joined) is two, (m = k, lo = 0) and (m = 64 - k, lo = k).  Pending
// steps are always consecutive steps of the tile, `rows` of them, the first
// starting at record `first`; `split` says whether any is a split step.
// Only packed records form split steps (kRuns); in a batch of 32-byte
// records every run is a whole step, which len() and at() give as constants.
template <bool kRuns>
struct LinBatchT {
    std::uint32_t page1;
    std::uint32_t bytes;
    std::uint64_t issue;
    std::uint32_t rid;  // range id (kept by the apply pass, for hybrid sampling)
    std::uint32_t m;    // records of the run
    std::uint32_t lo;   // lane of its first record in its step
    std::size_t first;
    int n;
    int rows;
    bool split;

    __device__ __forceinline__ void push(std::uint32_t p1, std::uint64_t i0, std::uint32_t b0,
                                         std::size_t s, std::uint32_t r = 0)
    {
        if (n == 0) {
            first = s;
        }
        if (static_cast<int>(threadIdx.x) == n) {
            page1 = p1;
            bytes = b0;
            issue = i0;
            rid = r;
            m = kWave;
            lo = 0;
        }
        ++n;
        ++rows;
    }
    // A split step: lanes 0 .. k-1 read page pa - 1, lanes k .. 63 page pb - 1
    // (needs n <= 62).
    __device__ __forceinline__ void push_split(std::uint32_t pa, std::uint32_t pb, std::uint32_t k,
                                               std::uint64_t i0, std::uint32_t b0, std::size_t s,
                                               std::uint32_t ra, std::uint32_t rb)
    {
        if (n == 0) {
            first = s;
        }
        const int l = static_cast<int>(threadIdx.x);
        if (l == n || l == n + 1) {
            const bool second = l == n + 1;
            page1 = second ? pb : pa;
            bytes = b0;
            issue = i0;
            rid = second ? rb : ra;
            m = second ? kWave - k : k;
            lo = second ? k : 0u;
        }
        n += 2;
        ++rows;
        split = true;
    }
    // Appends a linear group's D steps (needs n <= 64 - D).
    template <int D>
    __device__ __forceinline__ void push_group(const GroupLin<D>& gl, std::size_t s,
                                               std::uint32_t r = 0)
    {
        if (n == 0) {
            first = s;
        }
        const int j = static_cast<int>(threadIdx.x) - n;
        // batch lane n + j takes step j from the group's lane j (every lane
        // takes part in the shuffles)
        const int src = j >= 0 && j < D ? j : 0;
        const std::uint32_t p1 =
            static_cast<std::uint32_t>(__shfl(static_cast<int>(gl.page1), src));
        const std::uint64_t i0 = shfl64(gl.issue, src);
        if (j >= 0 && j < D) {
            page1 = p1;
            issue = i0;
            bytes = gl.bytes;
            rid = r;
            m = kWave;
            lo = 0;
        }
        n += D;
        rows += D;
    }
    __device__ __forceinline__ void clear()
    {
        n = 0;
        rows = 0;
        split = false;
    }
    __device__ __forceinline__ std::uint32_t len() const { return kRuns ? m : kWave; }
    __device__ __forceinline__ std::uint32_t at() const { return kRuns ? lo : 0u; }
    __device__ __forceinline__ bool any_split() const { return kRuns && split; }
};

template <bool kRuns>
__device__ __forceinline__ LinBatchT<kRuns> empty_batch()
{
    LinBatchT<kRuns> b;
    b.page1 = 0;
    b.bytes = 0;
    b.issue = 0;
    b.rid = 0;
    b.m = kWave;
    b.lo = 0;
    b.first = 0;
    b.n = 0;
    b.rows = 0;
    b.split = false;
    return b;
}

// Lane grouping by key for one step: the previous lane of the same key
// (pred, -1 for the first), and the group's first and last lanes.  When every
// active lane has the same key (sequential streams) the ballot match is
// skipped.
struct Group {
    int pred, leader, last;
    bool uniform;  // every active lane has the same key (wave-uniform)
};

// Lanes whose key equals this lane's key, through a per-wave LDS table of
// lane masks (tab[key] is 0 between calls): every lane ORs its bit into its
// key's slot, reads the slot back, and clears it.  A wave's LDS operations
// complete in issue order, so each read sees every lane's bit and each clear
// follows every read.  Every lane of the wave must call it.
__device__ __forceinline__ std::uint64_t match_lds(std::uint64_t* tab, std::uint32_t key, bool m,
                                                   int lane)
{
    std::uint64_t peers = 0;
    if (m) {
        __hip_atomic_fetch_or(&tab[key], 1ull << lane, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (m) {
        peers = __hip_atomic_load(&tab[key], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (m) {
        __hip_atomic_store(&tab[key], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return peers;
}

__device__ __forceinline__ Group group_by(std::uint32_t key, std::uint32_t bits, bool m,
                                          std::uint64_t active, int lane,
                                          std::uint64_t* tab = nullptr)
{
    const int first = __ffsll(static_cast<long long>(active)) - 1;
    const std::uint32_t key0 = static_cast<std::uint32_t>(__shfl(static_cast<int>(key), first));
    Group g;
    std::uint64_t peers;
    g.uniform = __ballot(m && key == key0) == active;
    if (g.uniform) {
        peers = active;
    } else if (tab != nullptr) {
        peers = match_lds(tab, key, m, lane);
    } else {
        peers = match_key(key, bits, active);
    }
    const std::uint64_t below = peers & lanemask_lt(lane);
    g.pred = (m && below) ? 63 - __clzll(below) : -1;
    g.leader = m ? __ffsll(static_cast<long long>(peers)) - 1 : lane;
    g.last = m ? 63 - __clzll(peers) : lane;
    return g;
}

// Plane grouping of a batch of linear steps (lane k: step k, active lanes a
// prefix).  Steps on one media page share a plane.  Striping maps the page
// modulo C W D P = Rp one-to-one onto the planes (mixed-radix digits), so
// when the batch's pages never fall from lane to lane and span fewer than Rp
// pages, the runs of equal page are exactly the plane groups: one shuffle and
// two ballots instead of a ballot per key bit.  Otherwise, by key.
__device__ __forceinline__ Group group_plane_runs(const KArgs& a, std::uint32_t page1,
                                                  std::uint32_t key, bool m,
                                                  std::uint64_t active, int lane,
                                                  std::uint64_t* tab)
{
    const std::uint32_t prev =
        static_cast<std::uint32_t>(__shfl(static_cast<int>(page1), lane > 0 ? lane - 1 : 0));
    const int last_lane = 63 - __clzll(active);
    const std::uint32_t p0 = rfl32(page1);
    const std::uint32_t pl = rl32(page1, last_lane);
    const bool falls = m && lane > 0 && prev > page1;
    if (__ballot(falls) != 0 || pl - p0 >= a.Rp) {
        return group_by(key, a.pbits, m, active, lane, tab);
    }
    const bool head = m && (lane == 0 || prev != page1);
    const std::uint64_t heads = __ballot(head);
    const std::uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
    const std::uint64_t later = heads & ~upto;
    Group g;
    g.uniform = heads == 1ull;
    g.pred = (m && !head) ? lane - 1 : -1;
    g.leader = m ? 63 - __clzll(heads & upto) : lane;
    g.last = m ? (later != 0 ? __ffsll(static_cast<long long>(later)) - 2 : last_lane) : lane;
    return g;
}

__device__ __forceinline__ void scan_group(const Group& g, std::uint64_t& A, std::uint64_t& B,
                                           int lane)
{
    if (g.uniform) {
        wave_scan(A, B);
    } else {
        group_scan(A, B, g.pred, lane);
    }
}

// Scans a step's plane maps and channel maps.  When the narrow check passes
// both run in 32 bits relative to the step's time origin: as interleaved DPP
// scans when both are single-key steps, else as interleaved pointer-jumping
// group scans.  Otherwise each runs exactly in 64 bits.
__device__ __forceinline__ void scan_pair(const Group& gp, std::uint64_t& Ap, std::uint64_t& Bp,
                                          const Group& gc, std::uint64_t& Ac, std::uint64_t& Bc,
                                          const Dec& d, bool m, std::uint64_t active,
                                          std::uint64_t svc, std::uint64_t xfer, int lane)
{
    const Narrow nw = narrow_check(d, m, active, svc, xfer);
    if (nw.ok) {
        std::uint32_t ap = static_cast<std::uint32_t>(Ap);
        std::uint32_t bp = Bp == 0 ? 0u : static_cast<std::uint32_t>(Bp - nw.origin);
        std::uint32_t ac = static_cast<std::uint32_t>(Ac);
        std::uint32_t bc = Bc == 0 ? 0u : static_cast<std::uint32_t>(Bc - nw.origin);
        if (gp.uniform && gc.uniform) {
            wave_scan32x2(ap, bp, ac, bc);
        } else {
            group_scan32x2(ap, bp, gp.pred, ac, bc, gc.pred, lane);
        }
        Ap = ap;
        Bp = nw.origin + bp;
        Ac = ac;
        Bc = nw.origin + bc;
        return;
    }
    scan_group(gp, Ap, Bp, lane);
    scan_group(gc, Ac, Bc, lane);
}

__device__ __forceinline__ std::uint64_t plane_service(const KArgs& a, std::uint32_t bits,
                                                       bool hit)
{
    if ((bits & 1u) == 0) {
        return hit ? 0ull : a.read_ps;
    }
    if (bits & 4u) {
        return a.read_ps + a.program_ps;
    }
    return (bits & 2u) ? a.program_ps : 0ull;
}

// The range fences (r_nfence <= kMaxFences), a lane's share in registers:
// fetch_fences issues every load before store_fences writes any of them, so
// a tile's set-up waits for memory once rather than once per 64 fences.
constexpr int kFencesPerLane = static_cast<int>(kMaxFences) / kWave;

struct FenceRegs {
    std::uint64_t v[kFencesPerLane];
};

__device__ __forceinline__ FenceRegs fetch_fences(const KArgs& a, int lane)
{
    FenceRegs f;
#pragma unroll
    for (int k = 0; k < kFencesPerLane; ++k) {
        const std::uint32_t j = static_cast<std::uint32_t>(lane + k * kWave);
        f.v[k] = j < a.r_nfence ? a.r_base[static_cast<std::size_t>(j) * a.r_stride] : 0ull;
    }
    return f;
}

__device__ __forceinline__ void store_fences(const KArgs& a, const FenceRegs& f,
                                             std::uint64_t* fence, int lane)
{
#pragma unroll
    for (int k = 0; k < kFencesPerLane; ++k) {
        const std::uint32_t j = static_cast<std::uint32_t>(lane + k * kWave);
        if (j < a.r_nfence) {
            fence[j] = f.v[k];
        }
    }
}

__device__ __forceinline__ void load_fences(const KArgs& a, std::uint64_t* fence, int lane)
{
    store_fences(a, fetch_fences(a, lane), fence, lane);
}

// Step view of a batch of linear steps: lane k < n stands for step k, with
// lane 0's record of that step (plane and channel from the media page, the
// byte count the channel moves per record and its transfer time).
struct StepView {
    Dec d;
    bool m;
    std::uint64_t active;
    std::uint64_t x;  // transfer of one record
};

template <bool kR>
__device__ __forceinline__ StepView step_view(const KArgs& a, const std::uint64_t* xp,
                                              const LinBatchT<kR>& q, int lane)
{
    StepView v;
    v.m = lane < q.n;
    v.active = q.n == kWave ? ~0ull : ((1ull << q.n) - 1);
    v.d.cls = v.m ? kClsModeled : kClsInvalid;
    v.d.bits = 0;
    v.d.plane = 0;
    v.d.chan = 0;
    v.d.range_id = 0;
    v.d.page1 = q.page1;
    v.d.issue = q.issue;
    v.d.xbytes = a.transfer_page ? (1ull << a.page_shift) : q.bytes;
    v.d.xfer = 0;
    if (v.m) {
        stripe(a, static_cast<std::uint64_t>(q.page1) - 1, v.d);
    }
    v.x = v.m ? xfer_ps_lds(a, xp, v.d.xbytes) : 0ull;
    return v;
}

// The summary pass keeps its per-plane LDS state at slot pslot(plane) =
// plane ^ ((plane >> 5) & 31), a permutation within each aligned block of 32
// planes (the arrays are padded to whole blocks, plane_slots).  A batch of
// linear steps walks the striping's fastest axis: its planes lie 32 apart on
// the 16 x 8 x 4 geometry (8 apart on 8 x 4 x 2), so plain indexing puts every
// lane of a fold on one LDS bank; the swizzle spreads them over distinct ones.
__host__ __device__ __forceinline__ std::uint32_t plane_slots(const KArgs& a)
{
    return (a.Rp + 31u) & ~31u;
}
__device__ __forceinline__ std::uint32_t pslot(std::uint32_t plane)
{
    return plane ^ ((plane >> 5) & 31u);
}

// Issue order across a batch of linear steps (one issue time per step):
// every step's time must be at least the one before it, the first step's at
// least `last` (the last issue time the wave saw before the batch).
template <bool kR>
__device__ __forceinline__ void batch_order(const LinBatchT<kR>& q, int lane, std::uint64_t& last,
                                            bool& back)
{
    const std::uint64_t prev = shfl64(q.issue, lane == 0 ? 0 : lane - 1);
    back = back || __ballot(lane < q.n && q.issue < (lane == 0 ? last : prev)) != 0;
    last = readlane64(q.issue, q.n - 1);
}

// Folds a batch of linear runs into the tile summary: the per-record fold of
// the general path applied to whole runs.  A run of m records after another
// record of its plane has plane map (sense, issue + sense) -- its first record
// senses unless its page is the one the plane last read, the others hit; a
// run that holds the tile's first record on its plane records that record
// and folds the m - 1 hits after it, map (0, issue) (the identity for m = 1).
// The channel map of a run is (m x, issue + m x).  kGiven: page-register
// hits come per record from `hits` (two page registers, whole steps only):
// a step's first record hits as hits[] says, and a step that is the tile's
// first record on its plane records that hit in its class (bit 3), as the
// per-record path does.
template <bool kR, bool kGiven = false>
__device__ __forceinline__ void fold_summary(const KArgs& a, const std::uint64_t* xp,
                                             const LinBatchT<kR>& q, int lane, std::uint64_t* p_fi,
                                             std::uint64_t* p_rA, std::uint64_t* p_rB,
                                             std::uint64_t* c_A, std::uint64_t* c_B,
                                             std::uint32_t* p_f1, std::uint32_t* p_l1,
                                             std::uint8_t* p_fc, std::uint64_t* mt_p,
                                             std::uint64_t* mt_c,
                                             const std::uint8_t* hits = nullptr)
{
    static_assert(!(kR && kGiven), "given hits take whole steps only");
    const StepView v = step_view(a, xp, q, lane);
    const bool m = v.m;
    const std::uint32_t pkey = m ? v.d.plane : 0u;
    const std::uint32_t ckey = m ? v.d.chan : 0u;
    const Group gp = group_plane_runs(a, q.page1, pkey, m, v.active, lane, mt_p);
    const Group gc = group_by(ckey, a.cbits, m, v.active, lane, mt_c);
    const std::uint32_t pk = pslot(pkey);
    const std::uint32_t f1 = m ? p_f1[pk] : 0u;
    const std::uint32_t last_page = m ? p_l1[pk] : 0u;
    const bool has = f1 != 0;
    const bool tfirst = m && gp.pred < 0 && !has;
    std::uint32_t prev1 = static_cast<std::uint32_t>(
        __shfl(static_cast<int>(q.page1), gp.pred < 0 ? lane : gp.pred));
    if (gp.pred < 0) {
        prev1 = last_page;
    }
    bool hit0 = prev1 == q.page1;
    if constexpr (kGiven) {
        hit0 = m && hits[q.first + static_cast<std::size_t>(lane) * kWave] != 0;
    }
    const std::uint64_t ls = hit0 ? 0ull : a.read_ps;
    const std::uint64_t cx = q.len() * v.x;
    std::uint64_t Ap = 0, Bp = 0, Ac = 0, Bc = 0;
    if (m) {
        // a run that holds the tile's first record on its plane records that
        // one apart; the map of the run's others is (0, issue), the identity
        // when it has none
        Ap = tfirst ? 0ull : ls;
        Bp = tfirst ? (q.len() >= 2 ? q.issue : 0ull) : q.issue + ls;
        Ac = cx;
        Bc = q.issue + cx;
    }
    scan_pair(gp, Ap, Bp, gc, Ac, Bc, v.d, m, v.active, ls, cx, lane);
    const std::uint32_t l1 =
        static_cast<std::uint32_t>(__shfl(static_cast<int>(q.page1), gp.leader));
    const std::uint64_t li = shfl64(q.issue, gp.leader);
    std::uint32_t lc = 0;  // the leader's class: a read (bit 3: its given hit)
    if constexpr (kGiven) {
        lc = static_cast<std::uint32_t>(__shfl(hit0 ? 8 : 0, gp.leader));
    }
    if (m && lane == gp.last) {
        if (!has) {
            p_f1[pk] = l1;
            p_fi[pk] = li;
            p_fc[pk] = static_cast<std::uint8_t>(lc);
        }
        const std::uint64_t sA = p_rA[pk];
        const std::uint64_t sB = p_rB[pk];
        p_rB[pk] = umax64(sB + Ap, Bp);
        p_rA[pk] = sA + Ap;
        p_l1[pk] = q.page1;
    }
    if (m && lane == gc.last) {
        const std::uint64_t sA = c_A[ckey];
        const std::uint64_t sB = c_B[ckey];
        c_B[ckey] = umax64(sB + Ac, Bc);
        c_A[ckey] = sA + Ac;
    }
}

// Writes a folded batch's step descriptors.  The summary pass calls it just
// before issuing a group's loads: vector memory operations complete in
// issue order, so a store placed after a group's loads would hold up the
// wait for that group.
template <bool kR>
__device__ __forceinline__ void write_descs(StepDesc* desc, SplitDesc* split, std::uint32_t* rid,
                                            LinBatchT<kR>& dq, int lane)
{
    if (dq.n != 0 && desc != nullptr) {
        // one descriptor per step, written by its first run's lane; a split
        // step's second run is the next lane
        // (32-byte batches hold whole steps only: row = lane, no second runs)
        const bool head = lane < dq.n && dq.at() == 0;
        const int row = kR ? __popcll(__ballot(head) & lanemask_lt(lane)) : lane;
        const int nx = lane + 1 < kWave ? lane + 1 : lane;
        std::uint32_t nlo = 0, np1 = 0, nrid = 0;
        if constexpr (kR) {
            nlo = static_cast<std::uint32_t>(__shfl(static_cast<int>(dq.at()), nx));
            np1 = static_cast<std::uint32_t>(__shfl(static_cast<int>(dq.page1), nx));
            nrid = static_cast<std::uint32_t>(__shfl(static_cast<int>(dq.rid), nx));
        }
        const bool second = kR && head && lane + 1 < dq.n && nlo != 0;
        if (head) {
            const std::size_t at = dq.first / kWave + static_cast<std::size_t>(row);
            StepDesc sd;
            sd.page1 = dq.page1;
            sd.bytes = dq.bytes | (second ? kSplitFlag : 0u);
            sd.issue = dq.issue;
            if (second && split == nullptr) {
                sd = StepDesc{0, 0, 0};  // no side array: replayed from its records
            }
            desc[at] = sd;
            if (second && split != nullptr) {
                split[at] = SplitDesc{np1, nlo, nrid, 0u};
            }
            if (rid != nullptr) {
                rid[at] = dq.rid;
            }
        }
    }
    dq.clear();
}

// 64-bit words of a tile's touched-plane mask.
__host__ __device__ __forceinline__ std::uint32_t mask_words(const KArgs& a)
{
    return (a.Rp + 63) / 64;
}

// A tile's plane summaries are packed: word w of its mask holds the touched
// planes r in [64 w, 64 w + 64) and how many touched planes come before them.
struct alignas(16) MaskWord {
    std::uint64_t bits;
    std::uint32_t base;
    std::uint32_t pad;
};

// Where plane r's entry sits among tile `tile`'s packed summaries (and carry-
// ins), or -1 when the tile does not touch the plane.
__device__ __forceinline__ int slot(const MaskWord* tmask, std::uint32_t words, std::size_t tile,
                                    std::uint32_t r)
{
    const MaskWord m = tmask[tile * words + r / 64];
    const std::uint32_t bit = r % 64;
    if (((m.bits >> bit) & 1u) == 0) {
        return -1;
    }
    return static_cast<int>(m.base) + __popcll(m.bits & ((1ull << bit) - 1));
}

// Byte offset of the summary pass's lane-matching tables (plane table, then
// channel table) after its state: fences, three 64-bit and two 32-bit plane
// arrays, two 64-bit channel arrays and the plane class bytes; 8-byte aligned.
__host__ __device__ __forceinline__ std::size_t summary_match_offset(const KArgs& a)
{
    const std::uint64_t rp = plane_slots(a);
    return 8ull * (a.r_nfence + 3ull * rp + 2ull * a.Rc) + 8ull * rp + ((rp + 7ull) & ~7ull);
}

// Byte offset of the summary pass's stripe table (Rp words), after the
// lane-matching tables when the run keeps them.
__host__ __device__ __forceinline__ std::size_t summary_stripe_offset(const KArgs& a)
{
    return summary_match_offset(a) + (a.match_lds ? 8ull * (a.Rp + a.Rc) : 0ull);
}

// Summary pass.  Per plane the tile keeps: the first record (page, issue,
// class), the (max,+) map of the records after it, and the last page; per
// channel the map of all its records.  Pages are stored as page + 1 in 32
// bits (capacity / page_bytes < 2^32 is checked on the host).
template <bool kRefresh, bool kHits, bool kPacked = false, bool kDeep = false, bool kFew = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kPacked ? (kDeep ? 2 : (kFew ? 3 : 4)) : 1))) void k_summary(KArgs a, const void* rec, std::size_t n,
                                                std::uint64_t base_ps, PlaneSum* psum,
                                                MaskWord* tmask, ChanSum* csum,
                                                std::uint64_t* tile_count,
                                                const std::uint8_t* hits, StepDesc* desc)
{
    extern __shared__ std::uint64_t sm[];
    // per-plane state at slot pslot(plane) of plane_slots(a) entries
    const std::uint32_t rpp = plane_slots(a);
    std::uint64_t* fence = sm;
    std::uint64_t* p_fi = fence + a.r_nfence;
    std::uint64_t* p_rA = p_fi + rpp;
    std::uint64_t* p_rB = p_rA + rpp;
    std::uint64_t* c_A = p_rB + rpp;
    std::uint64_t* c_B = c_A + a.Rc;
    std::uint32_t* p_f1 = reinterpret_cast<std::uint32_t*>(c_B + a.Rc);
    std::uint32_t* p_l1 = p_f1 + rpp;
    std::uint8_t* p_fc = reinterpret_cast<std::uint8_t*>(p_l1 + rpp);  // class bits < 16
    std::uint64_t* mt_p = a.match_lds ? reinterpret_cast<std::uint64_t*>(
                                            reinterpret_cast<unsigned char*>(sm) +
                                            summary_match_offset(a))
                                      : nullptr;
    std::uint64_t* mt_c = a.match_lds ? mt_p + a.Rp : nullptr;
    __shared__ std::uint64_t xp[33];
    const int lane = threadIdx.x;
    const std::size_t tile = blockIdx.x;
    const std::size_t begin = tile * a.tile;
    const std::size_t end = begin + a.tile < n ? begin + a.tile : n;
    // set-up loads and the first group of records are in flight together
    const FenceRegs fr = fetch_fences(a, lane);
    const std::uint64_t xv = fetch_xfer(a, lane);
    // The record before the tile: every record's issue time must be at least
    // its predecessor's for stream position to be the service order.  Steps
    // check their records against the last issue time seen (wave-uniform);
    // any that goes back sets a.disorder.
    std::uint64_t last_issue = 0;
    if (begin > 0) {
        last_issue = base_ps + (kPacked ? (static_cast<const hbf_record16*>(rec)[begin - 1].issue_op &
                                           ((1ull << 56) - 1))
                                        : static_cast<const hbf_record32*>(rec)[begin - 1].issue_ps);
    }
    bool disorder = false;
    bool any_split = false;  // some step of the tile was split (wave-uniform)
    // (the page-register variant takes no linear groups and keeps 4 deep;
    // packed records keep kPackedSumPipe steps at four waves per SIMD)
    // (kDeep: packed records where LDS already holds the pass at two waves
    // per SIMD, whose registers then allow 2 * kSumPipe steps in flight)
    constexpr int kDepth =
        kHits ? kPipe
              : (kDeep ? 2 * kSumPipe : (kPacked && !kFew ? kPackedSumPipe : kSumPipe));
    constexpr std::size_t kSpan = static_cast<std::size_t>(kDepth) * kWave;
    using Pipe = std::conditional_t<kPacked, PackedPipeT<kDepth>, RecordPipeT<kDepth>>;
    Pipe pipe;
    pipe.issue(rec, begin, end, lane);
    store_fences(a, fr, fence, lane);
    store_xfer(xp, xv, lane);
    for (std::uint32_t r = lane; r < rpp; r += kWave) {
        p_fi[r] = 0;
        p_rA[r] = 0;
        p_rB[r] = 0;
        p_f1[r] = 0;
        p_l1[r] = 0;
        p_fc[r] = 0;
    }
    for (std::uint32_t r = lane; r < a.Rc; r += kWave) {
        c_A[r] = 0;
        c_B[r] = 0;
    }
    if (a.match_lds) {
        for (std::uint32_t r = lane; r < a.Rp + a.Rc; r += kWave) {
            mt_p[r] = 0;
        }
    }
    std::uint32_t* stab = nullptr;
    if (a.stripe_lds) {
        stab = reinterpret_cast<std::uint32_t*>(reinterpret_cast<unsigned char*>(sm) +
                                                summary_stripe_offset(a));
        fill_stripe_table(a, stab, lane);
    }
    __syncthreads();
    RangeCache rc = empty_cache();
    RangeCache rcu = empty_cache();  // wave-uniform copy for linear steps
    LinBatchT<kPacked> q = empty_batch<kPacked>();
    LinBatchT<kPacked> dq = empty_batch<kPacked>();  // folded, descriptors not written yet
    // a batch is folded once it holds kFull runs: packed batches keep two
    // lanes free for a split step's runs
    constexpr int kFull = kPacked ? kWave - 1 : kWave;
    std::uint64_t modeled = 0;
    std::uint32_t lin_miss = 0;  // steps in a row that were not linear (wave-uniform)
    // descriptors of steps replayed from their records are zeroed up to 64
    // at a time, one lane per step: steps zbase + l for the bits l of zmask
    std::size_t zbase = 0;
    std::uint64_t zmask = 0;
    const auto flush_zero = [&]() {
        if (((zmask >> lane) & 1u) != 0) {
            desc[zbase + lane] = StepDesc{0, 0, 0};
        }
        zmask = 0;
    };
    for (std::size_t g = begin; g < end; g += kSpan) {
        pipe.promote();
        write_descs(desc, a.desc_split, a.desc_rid, dq, lane);
        if (g + kSpan < end) {
            pipe.issue(rec, g + kSpan, end, lane);
        }
        const std::size_t gend = g + kSpan < end ? g + kSpan : end;
        if ((kHits || a.slots == 1) && a.lead == nullptr && g + kSpan <= end &&
            q.n <= kWave - kDepth && lin_miss < kLinGiveUp) {
            // a whole group of linear steps joins the batch at once
            GroupLin<kDepth> gl;
            if (group_linear<kRefresh>(a, fence, rcu, pipe, base_ps, lane, gl)) {
                q.push_group(gl, g, rcu.id);
                if (q.n >= kFull || gend >= end) {
                    batch_order(q, lane, last_issue, disorder);
                    fold_summary<kPacked, kHits>(a, xp, q, lane, p_fi, p_rA, p_rB, c_A, c_B,
                                                 p_f1, p_l1, p_fc, mt_p, mt_c, hits);
                    modeled += static_cast<std::uint64_t>(q.rows) * kWave;
                    dq = q;  // (its descriptors wait for the next group's loads)
                    q.clear();
                }
                continue;
            }
        }
        for (std::size_t s = g; s < gend; s += kWave) {
            typename Pipe::Step st;
            pipe.take(st);
            const std::size_t i = s + lane;
            const bool valid = i < end;
            if ((kHits || a.slots == 1) && a.lead == nullptr) {
                // linear steps wait in a batch; the batch is folded when full, at
                // the tile's last step, and before any other step (order matters)
                LinStep ls;
                bool lin = false;
                if (lin_miss < kLinGiveUp || (s / kWave) % kLinProbe == 0) {
                    lin = detect_step<kRefresh, kPacked>(a, fence, rcu, st, base_ps, s + kWave <= end,
                                                lane, ls);
                    lin_miss = lin ? 0u : lin_miss + 1u;
                }
                if (lin) {
                    if (ls.k == 0) {
                        q.push(ls.page1, ls.issue, ls.bytes, s, ls.rid);
                    } else {
                        q.push_split(ls.page1, ls.page1b, ls.k, ls.issue, ls.bytes, s, ls.rid,
                                     ls.ridb);
                        any_split = true;
                    }
                }
                if (q.n != 0 && (!lin || q.n >= kFull || s + kWave >= end)) {
                    batch_order(q, lane, last_issue, disorder);
                    fold_summary<kPacked, kHits>(a, xp, q, lane, p_fi, p_rA, p_rB, c_A, c_B,
                                                 p_f1, p_l1, p_fc, mt_p, mt_c, hits);
                    modeled += static_cast<std::uint64_t>(q.rows) * kWave;
                    write_descs(desc, a.desc_split, a.desc_rid, dq, lane);  // at most one waits
                    dq = q;
                    q.clear();
                }
                if (lin) {
                    continue;
                }
                if (desc != nullptr) {  // replayed from its records
                    const std::size_t step = s / kWave;
                    if (zmask != 0 && step - zbase >= static_cast<std::size_t>(kWave)) {
                        flush_zero();
                    }
                    if (zmask == 0) {
                        zbase = step;
                    }
                    zmask |= 1ull << (step - zbase);
                }
            }
            uint4 x, y;
            step_records(st, lane, x, y);
            Dec d = valid ? decode<kRefresh>(a, fence, rc, x, y, base_ps, stab) : invalid_dec();
            {
                const std::uint64_t prev = shfl64(d.issue, lane == 0 ? 0 : lane - 1);
                const bool back = valid && d.issue < (lane == 0 ? last_issue : prev);
                disorder = disorder || __ballot(back) != 0;
                const std::uint64_t vmask = __ballot(valid);  // lanes 0 .. k
                last_issue = readlane64(d.issue, 63 - __clzll(static_cast<long long>(vmask)));
            }
            if (!kPacked && a.lead != nullptr && valid && a.lead[i] != 0) {
                d.cls = kClsFollower;
            }
            const bool m = valid && d.cls == kClsModeled;
            const bool hbit = kHits && valid && hits[i] != 0;
            const std::uint64_t active = __ballot(m);
            modeled += __popcll(active);
            if (active == 0) {
                continue;
            }
            const std::uint64_t xfer = lane_xfer(a, xp, d, m, active);
            if (!kHits && run_step(a, d, active, lane)) {
                const std::uint64_t W = run_channel_max(d, xfer, lane);
                if (lane == 63) {
                    const std::uint32_t pkey = pslot(d.plane);
                    const std::uint32_t ckey = d.chan;
                    const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
                    const std::uint64_t i0 = readlane64(d.issue, 0);
                    if (p_f1[pkey] == 0) {  // lane 0 is the tile's first record here
                        p_f1[pkey] = page1;
                        p_fi[pkey] = i0;
                        p_fc[pkey] = 0;
                        p_rA[pkey] = 0;
                        p_rB[pkey] = d.issue;
                    } else {
                        const bool lhit = p_l1[pkey] == page1;
                        const std::uint64_t ls = lhit ? 0ull : a.read_ps;
                        const std::uint64_t sA = p_rA[pkey] + ls;
                        const std::uint64_t sB = umax64(p_rB[pkey] + ls, i0 + ls);
                        p_rA[pkey] = sA;
                        p_rB[pkey] = umax64(sB, d.issue);
                    }
                    p_l1[pkey] = page1;
                    const std::uint64_t tA = 64 * xfer;
                    const std::uint64_t tB = W + xfer;
                    const std::uint64_t sA = c_A[ckey];
                    const std::uint64_t sB = c_B[ckey];
                    c_B[ckey] = umax64(sB + tA, tB);
                    c_A[ckey] = sA + tA;
                }
                continue;
            }
            const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
            const std::uint32_t pkey = m ? d.plane : 0u;
            const std::uint32_t ckey = m ? d.chan : 0u;
            const Group gp = group_by(pkey, a.pbits, m, active, lane, mt_p);
            const Group gc = group_by(ckey, a.cbits, m, active, lane, mt_c);
            // state reads come before this step's writes
            const std::uint32_t pk = pslot(pkey);
            const std::uint32_t f1 = m ? p_f1[pk] : 0u;
            const std::uint32_t last_page = m ? p_l1[pk] : 0u;
            const bool has = f1 != 0;
            const bool tfirst = m && gp.pred < 0 && !has;
            std::uint32_t prev1 = static_cast<std::uint32_t>(
                __shfl(static_cast<int>(page1), gp.pred < 0 ? lane : gp.pred));
            if (gp.pred < 0) {
                prev1 = last_page;
            }
            const bool hit = kHits ? (m && hbit) : (a.slots != 0 && m && prev1 == page1);
            const std::uint64_t svc = plane_service(a, d.bits, hit);
            std::uint64_t Ap = 0, Bp = 0;
            if (m && !tfirst) {
                Ap = svc;
                Bp = d.issue + svc;
            }
            std::uint64_t Ac = m ? xfer : 0ull;
            std::uint64_t Bc = m ? d.issue + xfer : 0ull;
            scan_pair(gp, Ap, Bp, gc, Ac, Bc, d, m, active, svc, xfer, lane);
            const std::uint32_t l1 =
                static_cast<std::uint32_t>(__shfl(static_cast<int>(page1), gp.leader));
            const std::uint64_t li = shfl64(d.issue, gp.leader);
            // the leader's class; with given hits, bit 3 carries its hit
            const std::uint32_t lbits = kHits && hit ? (d.bits | 8u) : d.bits;
            const std::uint32_t lc =
                static_cast<std::uint32_t>(__shfl(static_cast<int>(lbits), gp.leader));
            if (m && lane == gp.last) {
                if (!has) {
                    p_f1[pk] = l1;
                    p_fi[pk] = li;
                    p_fc[pk] = static_cast<std::uint8_t>(lc);
                }
                const std::uint64_t sA = p_rA[pk];
                const std::uint64_t sB = p_rB[pk];
                p_rB[pk] = umax64(sB + Ap, Bp);
                p_rA[pk] = sA + Ap;
                p_l1[pk] = page1;
            }
            if (m && lane == gc.last) {
                const std::uint64_t sA = c_A[ckey];
                const std::uint64_t sB = c_B[ckey];
                c_B[ckey] = umax64(sB + Ac, Bc);
                c_A[ckey] = sA + Ac;
            }
        }
    }
    write_descs(desc, a.desc_split, a.desc_rid, dq, lane);
    if (desc != nullptr) {
        flush_zero();
    }
    if (disorder && a.disorder != nullptr && lane == 0) {
        *a.disorder = 1u;
    }
    if (kPacked && a.tile_split != nullptr && lane == 0) {
        a.tile_split[tile] = any_split ? 1u : 0u;
    }
    __syncthreads();
    // Only planes the tile touched get a summary, packed in plane order; the
    // tile's mask words say which (the others are identities, and the carry
    // chain skips them).
    PlaneSum* ps = psum + tile * a.Rp;
    MaskWord* tm = tmask + tile * mask_words(a);
    std::uint32_t count = 0;
    for (std::uint32_t r0 = 0; r0 < a.Rp; r0 += kWave) {
        const std::uint32_t r = r0 + lane;
        const std::uint32_t k = pslot(r);
        const bool touched = r < a.Rp && p_f1[k] != 0;
        const std::uint64_t bits = __ballot(touched);
        if (lane == 0) {
            MaskWord m;
            m.bits = bits;
            m.base = count;
            m.pad = 0;
            tm[r0 / kWave] = m;
        }
        if (touched) {
            PlaneSum v;
            v.fpage1 = p_f1[k];
            v.fissue = p_fi[k];
            v.rA = p_rA[k];
            v.rB = p_rB[k];
            v.lpage1 = p_l1[k];
            v.fcls = p_fc[k];
            v.pad = 0;
            ps[count + __popcll(bits & lanemask_lt(lane))] = v;
        }
        count += static_cast<std::uint32_t>(__popcll(bits));
    }
    ChanSum* cs = csum + tile * a.Rc;
    for (std::uint32_t r = lane; r < a.Rc; r += kWave) {
        ChanSum v;
        v.A = c_A[r];
        v.B = c_B[r];
        cs[r] = v;
    }
    if (lane == 0) {
        tile_count[tile] = modeled;
    }
}

__device__ __forceinline__ void add128(std::uint64_t& lo, std::uint64_t& hi, std::uint64_t v)
{
    const std::uint64_t n = lo + v;
    hi += n < lo ? 1u : 0u;
    lo = n;
}

__device__ __forceinline__ std::uint64_t wave_sum(std::uint64_t v)
{
    for (int o = 32; o > 0; o >>= 1) {
        v += shfl64(v, threadIdx.x ^ o);
    }
    return v;
}

// ---- carry chain: a three-level scan over tile summaries ---------------
//
// A plane summary is a (first record, (max,+) map of the rest, last page)
// triple.  Two summaries compose associatively: the later summary's first
// record resolves its page-register hit against the earlier one's last page,
// then joins the map.  Level 1 folds groups of kGroup tiles, level 2 walks
// the groups of each resource in order from the engine state, level 3 walks
// each group's tiles from the group's carry-in.  One thread per (group,
// resource) at levels 1 and 3, one per resource at level 2.

constexpr std::uint32_t kGroup = 16;
constexpr int kChunk = 8;  // loads a carry thread keeps in flight

__device__ __forceinline__ PlaneSum plane_compose(const KArgs& a, const PlaneSum& s1,
                                                  const PlaneSum& s2)
{
    if (s2.fpage1 == 0) {
        return s1;
    }
    if (s1.fpage1 == 0) {
        return s2;
    }
    PlaneSum r = s1;
    const bool hit = a.ext_hits ? (s2.fcls & 8u) != 0 : (a.slots != 0 && s2.fpage1 == s1.lpage1);
    const std::uint64_t svc = plane_service(a, s2.fcls, hit);
    // rest1, then the later first record (svc, issue + svc), then rest2; A
    // is also the service total of the records after the first
    const std::uint64_t A = s1.rA + svc;
    const std::uint64_t B = umax64(s1.rB + svc, s2.fissue + svc);
    r.rB = umax64(B + s2.rA, s2.rB);
    r.rA = A + s2.rA;
    r.lpage1 = s2.lpage1;
    return r;
}

// Applies a summary to a plane's state; returns the service it charged.
__device__ __forceinline__ std::uint64_t plane_apply(const KArgs& a, const PlaneSum& s,
                                                     std::uint64_t& busy, std::uint64_t& tag1)
{
    if (s.fpage1 == 0) {
        return 0;
    }
    const bool hit = a.ext_hits ? (s.fcls & 8u) != 0 : (a.slots != 0 && tag1 == s.fpage1);
    const std::uint64_t svc = plane_service(a, s.fcls, hit);
    if (a.contention) {
        const std::uint64_t b = umax64(busy, s.fissue) + svc;
        busy = umax64(b + s.rA, s.rB);
    }
    tag1 = s.lpage1;
    return svc + s.rA;
}

__device__ __forceinline__ ChanSum chan_compose(const ChanSum& s1, const ChanSum& s2)
{
    ChanSum r;
    r.A = s1.A + s2.A;
    r.B = umax64(s1.B + s2.A, s2.B);
    return r;
}

// Level 1: thread (g, r) folds the summaries of group g's tiles.
// Slots of plane r in tiles t .. t + kChunk - 1 (those below t1; -1 where
// a tile did not touch r).  The chunk's mask words are loaded whole and
// together before any is decoded: decoding each word as it arrives would
// put a memory round trip per tile in front of the summaries' loads.
__device__ __forceinline__ void chunk_slots(const MaskWord* tmask, std::uint32_t words,
                                            std::size_t t, std::size_t t1, std::uint32_t r,
                                            int (&at)[kChunk])
{
    MaskWord mw[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        mw[k] = t + k < t1 ? tmask[(t + k) * words + r / 64] : MaskWord{0, 0, 0};
    }
    const std::uint32_t bit = r % 64;
    const std::uint64_t below = (1ull << bit) - 1;
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        at[k] = ((mw[k].bits >> bit) & 1u) != 0
                    ? static_cast<int>(mw[k].base) + __popcll(mw[k].bits & below)
                    : -1;
    }
}

// Level-1 work of thread (g, r): the composition of group g's tile
// summaries of plane r, of channel c, and its tiles' modeled-record count.
// Loads go out kChunk at a time ahead of the (serial) composition, so a
// thread waits once per chunk rather than once per tile.
__device__ __forceinline__ PlaneSum plane_fold(const KArgs& a, const PlaneSum* psum,
                                               const MaskWord* tmask, std::size_t ntiles,
                                               std::size_t g, std::uint32_t r)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    const std::uint32_t words = mask_words(a);
    PlaneSum acc{};  // the identity: no first record
#pragma unroll
    for (std::uint32_t c = 0; c < kGroup / kChunk; ++c) {
        const std::size_t t = t0 + static_cast<std::size_t>(c) * kChunk;
        if (t >= t1) {
            break;
        }
        int at[kChunk];
        PlaneSum buf[kChunk];
        chunk_slots(tmask, words, t, t1, r, at);
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (at[k] >= 0) {
                buf[k] = psum[(t + k) * a.Rp + at[k]];
            }
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (at[k] >= 0) {
                acc = plane_compose(a, acc, buf[k]);
            }
        }
    }
    return acc;
}

__device__ __forceinline__ ChanSum chan_fold(const KArgs& a, const ChanSum* csum,
                                             std::size_t ntiles, std::size_t g, std::uint32_t c)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    ChanSum acc{0, 0};  // the identity
    for (std::size_t t = t0; t < t1; t += kChunk) {
        ChanSum buf[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            buf[k] = t + k < t1 ? csum[(t + k) * a.Rc + c] : ChanSum{0, 0};
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            acc = chan_compose(acc, buf[k]);
        }
    }
    return acc;
}

__device__ __forceinline__ std::uint64_t count_fold(const std::uint64_t* tile_count,
                                                    std::size_t ntiles, std::size_t g)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    std::uint64_t sum = 0;
    for (std::size_t t = t0; t < t1; ++t) {
        sum += tile_count[t];
    }
    return sum;
}

__global__ __launch_bounds__(256) void k_carry_up(KArgs a, std::size_t ntiles, std::size_t ngroups,
                                                  const PlaneSum* psum,
                                                  const MaskWord* tmask, const ChanSum* csum,
                                                  const std::uint64_t* tile_count,
                                                  PlaneSum* gpsum, ChanSum* gcsum,
                                                  std::uint64_t* gcount)
{
    const std::uint32_t rt = a.Rp + a.Rc + 1;
    const std::size_t id = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= ngroups * rt) {
        return;
    }
    const std::size_t g = id / rt;
    const std::uint32_t r = static_cast<std::uint32_t>(id - g * rt);
    if (r < a.Rp) {
        gpsum[g * a.Rp + r] = plane_fold(a, psum, tmask, ntiles, g, r);
    } else if (r < a.Rp + a.Rc) {
        const std::uint32_t c = r - a.Rp;
        gcsum[g * a.Rc + c] = chan_fold(a, csum, ntiles, g, c);
    } else {
        gcount[g] = count_fold(tile_count, ntiles, g);
    }
}

// Level 2: block r scans resource r's group summaries (an exclusive scan by
// composition, kMidBlock groups per pass with a running carry) and applies
// each prefix to the engine state: every group's carry-in, the final state,
// and the service total.
constexpr int kMidBlock = 512;
// runs of at most this many tiles take the one-launch chain (k_carry_one)
constexpr std::size_t kOneCarryTiles = static_cast<std::size_t>(kMidBlock) * kChunk;

// one entry per wave of the block: the waves' inclusive totals
union MidShared {
    PlaneSum p[kMidBlock / kWave];
    ChanSum c[kMidBlock / kWave];
    std::uint64_t s[kMidBlock / kWave];
};

// Lane `src`'s value of a scanned type.
__device__ __forceinline__ std::uint64_t lane_value(std::uint64_t v, int src)
{
    return shfl64(v, src);
}

__device__ __forceinline__ ChanSum lane_value(const ChanSum& v, int src)
{
    return ChanSum{shfl64(v.A, src), shfl64(v.B, src)};
}

__device__ __forceinline__ PlaneSum lane_value(const PlaneSum& v, int src)
{
    PlaneSum r;
    r.fpage1 = shfl64(v.fpage1, src);
    r.fissue = shfl64(v.fissue, src);
    r.rA = shfl64(v.rA, src);
    r.rB = shfl64(v.rB, src);
    r.lpage1 = shfl64(v.lpage1, src);
    r.fcls = static_cast<std::uint32_t>(__shfl(static_cast<int>(v.fcls), src));
    r.pad = 0;
    return r;
}

// Inclusive scan of x over the block, earlier elements first: each wave
// scans its lanes through shuffles (Hillis-Steele), then every thread
// composes the totals of the waves before its own from LDS; two barriers in
// all.  `excl` receives the exclusive prefix (identity for thread 0).
template <typename T, typename F>
__device__ __forceinline__ T block_scan(T x, T* wsh, T identity, F compose, T& excl)
{
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int w = tid / kWave;
    for (int off = 1; off < kWave; off <<= 1) {
        const T y = lane_value(x, lane >= off ? lane - off : lane);
        if (lane >= off) {
            x = compose(y, x);
        }
    }
    T before_lane = lane_value(x, lane > 0 ? lane - 1 : 0);
    if (lane == kWave - 1) {
        wsh[w] = x;
    }
    __syncthreads();
    T before = identity;
    for (int k = 0; k < w; ++k) {
        before = compose(before, wsh[k]);
    }
    __syncthreads();  // (wsh may be written again after the return)
    excl = lane > 0 ? compose(before, before_lane) : before;
    return compose(before, x);
}

__device__ __forceinline__ std::uint64_t block_sum(std::uint64_t v, std::uint64_t* sh)
{
    const std::uint64_t w = wave_sum(v);
    const int tid = threadIdx.x;
    if ((tid & (kWave - 1)) == 0) {
        sh[tid / kWave] = w;
    }
    __syncthreads();
    std::uint64_t total = 0;
    for (int k = 0; k < kMidBlock / kWave; ++k) {
        total += sh[k];
    }
    __syncthreads();
    return total;
}

__global__ __launch_bounds__(kMidBlock) void k_carry_mid(
    KArgs a, std::size_t ngroups, const PlaneSum* gpsum, const ChanSum* gcsum,
    const std::uint64_t* gcount, PlaneCarry* gpcarry, std::uint64_t* gccarry,
    std::uint64_t* gseq, std::uint64_t* st_pbusy, std::uint64_t* st_ptag,
    std::uint64_t* st_cbusy, std::uint64_t* st_seq, std::uint64_t* ptotal, std::uint64_t* ctotal)
{
    __shared__ MidShared sh;
    __shared__ std::uint64_t red[kMidBlock / kWave];
    __shared__ std::uint64_t next[2];
    const std::uint32_t r = blockIdx.x;
    const int tid = threadIdx.x;
    // a stream whose issue time goes back is timed again from a sorted copy:
    // this run then leaves the engine state as it found it
    const bool commit = a.disorder == nullptr || *a.disorder == 0u;
    if (r < a.Rp) {
        std::uint64_t busy = st_pbusy[r];
        std::uint64_t tag1 = st_ptag[static_cast<std::size_t>(r) * 2];
        std::uint64_t total = 0;
        const PlaneSum id{};
        const auto compose = [&](const PlaneSum& s1, const PlaneSum& s2) {
            return plane_compose(a, s1, s2);
        };
        for (std::size_t g0 = 0; g0 < ngroups; g0 += kMidBlock) {
            const std::size_t g = g0 + tid;
            PlaneSum own = id;
            if (g < ngroups) {
                own = gpsum[g * a.Rp + r];
            }
            PlaneSum before;
            (void)block_scan(own, sh.p, id, compose, before);
            std::uint64_t b = busy, t1 = tag1;
            (void)plane_apply(a, before, b, t1);  // the state this group starts from
            std::uint64_t svc = 0;
            if (g < ngroups) {
                PlaneCarry c;
                c.busy = b;
                c.tag1 = t1;
                gpcarry[g * a.Rp + r] = c;
                svc = plane_apply(a, own, b, t1);
            }
            const std::size_t last = (ngroups - g0 < kMidBlock ? ngroups - g0 : kMidBlock) - 1;
            if (static_cast<std::size_t>(tid) == last) {
                next[0] = b;
                next[1] = t1;
            }
            total += block_sum(svc, red);
            busy = next[0];
            tag1 = next[1];
            __syncthreads();
        }
        if (tid == 0 && commit) {
            st_pbusy[r] = busy;
            st_ptag[static_cast<std::size_t>(r) * 2] = tag1;
            ptotal[r] += total;
        }
    } else if (r < a.Rp + a.Rc) {
        const std::uint32_t c = r - a.Rp;
        std::uint64_t busy = st_cbusy[c];
        std::uint64_t total = 0;
        const ChanSum id{0, 0};
        for (std::size_t g0 = 0; g0 < ngroups; g0 += kMidBlock) {
            const std::size_t g = g0 + tid;
            ChanSum own = id;
            if (g < ngroups) {
                own = gcsum[g * a.Rc + c];
            }
            ChanSum before;
            const ChanSum inc = block_scan(own, sh.c, id, chan_compose, before);
            if (g < ngroups) {
                gccarry[g * a.Rc + c] = umax64(busy + before.A, before.B);
            }
            const std::size_t last = (ngroups - g0 < kMidBlock ? ngroups - g0 : kMidBlock) - 1;
            if (static_cast<std::size_t>(tid) == last) {
                next[0] = umax64(busy + inc.A, inc.B);
            }
            total += block_sum(g < ngroups ? own.A : 0ull, red);
            busy = next[0];
            __syncthreads();
        }
        if (tid == 0 && commit) {
            st_cbusy[c] = busy;
            ctotal[c] += total;
        }
    } else if (r == a.Rp + a.Rc) {
        std::uint64_t seq = *st_seq;
        const auto add = [](std::uint64_t x, std::uint64_t y) { return x + y; };
        for (std::size_t g0 = 0; g0 < ngroups; g0 += kMidBlock) {
            const std::size_t g = g0 + tid;
            const std::uint64_t own = g < ngroups ? gcount[g] : 0ull;
            std::uint64_t before;
            const std::uint64_t inc = block_scan(own, sh.s, std::uint64_t{0}, add, before);
            if (g < ngroups) {
                gseq[g] = seq + before;
            }
            const std::size_t last = (ngroups - g0 < kMidBlock ? ngroups - g0 : kMidBlock) - 1;
            if (static_cast<std::size_t>(tid) == last) {
                next[0] = seq + inc;
            }
            __syncthreads();
            seq = next[0];
            __syncthreads();
        }
        if (tid == 0 && commit) {
            *st_seq = seq;
        }
    }
}

// Level-3 work of thread (g, r): walks group g's tiles from the group's
// carry-in and writes every tile's carry-in.
__device__ __forceinline__ void plane_walk(const KArgs& a, const PlaneSum* psum,
                                           const MaskWord* tmask, std::size_t ntiles,
                                           std::size_t g, std::uint32_t r, PlaneCarry c0,
                                           PlaneCarry* pcarry)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    const std::uint32_t words = mask_words(a);
    std::uint64_t busy = c0.busy, tag1 = c0.tag1;
#pragma unroll
    for (std::uint32_t c = 0; c < kGroup / kChunk; ++c) {
        const std::size_t t = t0 + static_cast<std::size_t>(c) * kChunk;
        if (t >= t1) {
            break;
        }
        int at[kChunk];
        PlaneSum buf[kChunk];
        chunk_slots(tmask, words, t, t1, r, at);
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (at[k] >= 0) {
                buf[k] = psum[(t + k) * a.Rp + at[k]];
            }
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            // an untouched tile neither reads nor changes this plane
            if (at[k] >= 0) {
                PlaneCarry c;
                c.busy = busy;
                c.tag1 = tag1;
                pcarry[(t + k) * a.Rp + at[k]] = c;  // packed like the summaries
                (void)plane_apply(a, buf[k], busy, tag1);
            }
        }
    }
}

__device__ __forceinline__ void chan_walk(const KArgs& a, const ChanSum* csum, std::size_t ntiles,
                                          std::size_t g, std::uint32_t c, std::uint64_t busy,
                                          std::uint64_t* ccarry)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    for (std::size_t t = t0; t < t1; t += kChunk) {
        ChanSum buf[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            buf[k] = t + k < t1 ? csum[(t + k) * a.Rc + c] : ChanSum{0, 0};
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (t + k < t1) {
                ccarry[(t + k) * a.Rc + c] = busy;
                busy = umax64(busy + buf[k].A, buf[k].B);
            }
        }
    }
}

__device__ __forceinline__ void seq_walk(const std::uint64_t* tile_count, std::size_t ntiles,
                                         std::size_t g, std::uint64_t s, std::uint64_t* tile_seq)
{
    const std::size_t t0 = g * kGroup;
    const std::size_t t1 = t0 + kGroup < ntiles ? t0 + kGroup : ntiles;
    for (std::size_t t = t0; t < t1; ++t) {
        tile_seq[t] = s;
        s += tile_count[t];
    }
}

// Level 3: thread (g, r) walks group g's tiles from the group carry-in.
__global__ __launch_bounds__(256) void k_carry_down(KArgs a, std::size_t ntiles,
                                                    std::size_t ngroups, const PlaneSum* psum,
                                                    const MaskWord* tmask,
                                                    const ChanSum* csum,
                                                    const std::uint64_t* tile_count,
                                                    const PlaneCarry* gpcarry,
                                                    const std::uint64_t* gccarry,
                                                    const std::uint64_t* gseq, PlaneCarry* pcarry,
                                                    std::uint64_t* ccarry, std::uint64_t* tile_seq)
{
    const std::uint32_t rt = a.Rp + a.Rc + 1;
    const std::size_t id = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= ngroups * rt) {
        return;
    }
    const std::size_t g = id / rt;
    const std::uint32_t r = static_cast<std::uint32_t>(id - g * rt);
    if (r < a.Rp) {
        plane_walk(a, psum, tmask, ntiles, g, r, gpcarry[g * a.Rp + r], pcarry);
    } else if (r < a.Rp + a.Rc) {
        const std::uint32_t c = r - a.Rp;
        chan_walk(a, csum, ntiles, g, c, gccarry[g * a.Rc + c], ccarry);
    } else {
        seq_walk(tile_count, ntiles, g, gseq[g], tile_seq);
    }
}

// The whole chain in one launch, for runs of at most kMidBlock * kChunk
// tiles.  Thread g of block r owns tiles [g span, g span + span) (span <=
// kChunk): it loads their summaries of resource r in one round, folds them,
// the block scans the folds from the engine state, and the thread walks its
// tiles from its carry-in with the summaries still in registers.  Two
// rounds of dependent loads in all, where the three kernels above take
// eight; the compositions, and so the results, are the same.
__global__ __launch_bounds__(kMidBlock) void k_carry_one(
    KArgs a, std::size_t ntiles, std::uint32_t span, const PlaneSum* psum,
    const MaskWord* tmask, const ChanSum* csum, const std::uint64_t* tile_count,
    PlaneCarry* pcarry, std::uint64_t* ccarry, std::uint64_t* tile_seq,
    std::uint64_t* st_pbusy, std::uint64_t* st_ptag, std::uint64_t* st_cbusy,
    std::uint64_t* st_seq, std::uint64_t* ptotal, std::uint64_t* ctotal)
{
    __shared__ MidShared sh;
    __shared__ std::uint64_t red[kMidBlock / kWave];
    const std::uint32_t r = blockIdx.x;
    const std::size_t t0 = static_cast<std::size_t>(threadIdx.x) * span;
    const std::size_t t1 = t0 + span < ntiles ? t0 + span : ntiles;
    const bool in = t0 < ntiles;
    const bool last = in && t1 == ntiles;
    const bool commit = a.disorder == nullptr || *a.disorder == 0u;
    if (r < a.Rp) {
        std::uint64_t busy = st_pbusy[r];
        std::uint64_t tag1 = st_ptag[static_cast<std::size_t>(r) * 2];
        const auto compose = [&](const PlaneSum& s1, const PlaneSum& s2) {
            return plane_compose(a, s1, s2);
        };
        int at[kChunk];
        PlaneSum buf[kChunk];
        chunk_slots(tmask, mask_words(a), t0, in ? t1 : t0, r, at);
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (at[k] >= 0) {
                buf[k] = psum[(t0 + k) * a.Rp + at[k]];
            }
        }
        PlaneSum own{};
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (at[k] >= 0) {
                own = compose(own, buf[k]);
            }
        }
        PlaneSum before;
        (void)block_scan(own, sh.p, PlaneSum{}, compose, before);
        (void)plane_apply(a, before, busy, tag1);  // the state this thread's tiles start from
        std::uint64_t svc = 0;
        {
            std::uint64_t b = busy, t = tag1;
            svc = plane_apply(a, own, b, t);
        }
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            // an untouched tile neither reads nor changes this plane
            if (at[k] >= 0) {
                pcarry[(t0 + k) * a.Rp + at[k]] = PlaneCarry{busy, tag1};
                (void)plane_apply(a, buf[k], busy, tag1);
            }
        }
        const std::uint64_t total = block_sum(svc, red);
        if (last && commit) {
            st_pbusy[r] = busy;
            st_ptag[static_cast<std::size_t>(r) * 2] = tag1;
        }
        if (threadIdx.x == 0 && commit) {
            ptotal[r] += total;
        }
    } else if (r < a.Rp + a.Rc) {
        const std::uint32_t c = r - a.Rp;
        std::uint64_t busy = st_cbusy[c];
        ChanSum buf[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            buf[k] = t0 + k < t1 ? csum[(t0 + k) * a.Rc + c] : ChanSum{0, 0};
        }
        ChanSum own{0, 0};
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            own = chan_compose(own, buf[k]);
        }
        ChanSum before;
        const ChanSum inc = block_scan(own, sh.c, ChanSum{0, 0}, chan_compose, before);
        const std::uint64_t fin = umax64(busy + inc.A, inc.B);
        busy = umax64(busy + before.A, before.B);
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (t0 + k < t1) {
                ccarry[(t0 + k) * a.Rc + c] = busy;
                busy = umax64(busy + buf[k].A, buf[k].B);
            }
        }
        const std::uint64_t total = block_sum(own.A, red);
        if (last && commit) {
            st_cbusy[c] = fin;
        }
        if (threadIdx.x == 0 && commit) {
            ctotal[c] += total;
        }
    } else if (r == a.Rp + a.Rc) {
        const std::uint64_t seq = *st_seq;
        std::uint64_t cnt[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            cnt[k] = t0 + k < t1 ? tile_count[t0 + k] : 0ull;
        }
        std::uint64_t own = 0;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            own += cnt[k];
        }
        std::uint64_t before;
        const std::uint64_t inc = block_scan(
            own, sh.s, std::uint64_t{0}, [](std::uint64_t x, std::uint64_t y) { return x + y; },
            before);
        std::uint64_t q = seq + before;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
            if (t0 + k < t1) {
                tile_seq[t0 + k] = q;
                q += cnt[k];
            }
        }
        if (last && commit) {
            *st_seq = seq + inc;
        }
    }
}


__device__ __forceinline__ std::uint64_t wave_max(std::uint64_t v)
{
    for (int o = 32; o > 0; o >>= 1) {
        v = umax64(v, shfl64(v, threadIdx.x ^ o));
    }
    return v;
}

// Replays a batch of linear steps from the plane and channel state and writes
// their completions.  Per step, lane 0 senses unless its page is the one the
// plane last read (with contention the plane is busy from max(busy, issue)
// for the sense, and the hits after it end at the same time); the channel
// moves the 64 records back to back from max(channel busy, issue).  The
// step-level maps are scanned across the batch exactly as records are in the
// general path; then every step's 64 completions follow in closed form:
//   plane  lane 0: lead = max(busy, issue) + sense (busy ignored without
//          contention); lanes 1..63: lead with contention, else issue;
//   channel lane j: top - x (63 - j), top = max(busy, issue) + 64 x.
struct ApplySums {
    std::uint64_t n_rec, n_mod, n_rd, n_hit, mk, lat_lo, lat_hi, lat_max, svc_sum, seq, n_hyb;
};

// kGiven: page-register hits per record from `given` (two page registers):
// a step's first record hits as given[] says.
template <bool kR, bool kGiven = false>
__device__ __forceinline__ void fold_apply(const KArgs& a, const std::uint64_t* xp,
                                           const LinBatchT<kR>& q, int lane, std::uint64_t* p_busy,
                                           std::uint64_t* c_busy, std::uint32_t* p_tag,
                                           std::uint64_t* completion, std::uint8_t* status,
                                           ApplySums& t, std::uint64_t* mt_p,
                                           std::uint64_t* mt_c, const std::uint8_t* given = nullptr)
{
    const StepView v = step_view(a, xp, q, lane);
    const bool m = v.m;
    const std::uint32_t pkey = m ? v.d.plane : 0u;
    const std::uint32_t ckey = m ? v.d.chan : 0u;
    const Group gp = group_plane_runs(a, q.page1, pkey, m, v.active, lane, mt_p);
    const Group gc = group_by(ckey, a.cbits, m, v.active, lane, mt_c);
    const std::uint32_t tag = m ? p_tag[pkey] : 0u;
    const std::uint64_t pbusy = m ? p_busy[pkey] : 0ull;
    const std::uint64_t cbusy = m ? c_busy[ckey] : 0ull;
    std::uint32_t prev1 = static_cast<std::uint32_t>(
        __shfl(static_cast<int>(q.page1), gp.pred < 0 ? lane : gp.pred));
    if (gp.pred < 0) {
        prev1 = tag;
    }
    bool lhit = m && prev1 == q.page1;
    if constexpr (kGiven) {
        lhit = m && given[q.first + static_cast<std::size_t>(lane) * kWave] != 0;
    }
    const std::uint64_t ls = lhit ? 0ull : a.read_ps;
    const std::uint64_t cx = 64 * v.x;
    std::uint64_t Ap = 0, Bp = 0, Ac = 0, Bc = 0;
    if (m) {
        Ap = ls;
        Bp = q.issue + ls;
        Ac = cx;
        Bc = q.issue + cx;
    }
    if (a.contention) {
        scan_pair(gp, Ap, Bp, gc, Ac, Bc, v.d, m, v.active, ls, cx, lane);
    } else {
        scan_group(gc, Ac, Bc, lane);
    }
    const std::uint64_t lead = a.contention ? umax64(pbusy + Ap, Bp) : q.issue + ls;
    const std::uint64_t top = umax64(cbusy + Ac, Bc);
    if (m && lane == gp.last) {
        if (a.contention) {
            p_busy[pkey] = lead;
        }
        p_tag[pkey] = q.page1;
    }
    if (m && lane == gc.last) {
        c_busy[ckey] = top;
    }
    // accounting: every lane gets one record of each step; all are modeled
    // reads, lanes 1..63 hit, lane 0 hits when its page was buffered
    const std::uint64_t nq = static_cast<std::uint64_t>(q.n);
    const std::uint64_t hits = __ballot(lhit);  // (every lane takes part)
    t.n_rec += nq;
    t.n_mod += nq;
    t.n_rd += nq;
    t.n_hit += lane == 0 ? static_cast<std::uint64_t>(__popcll(hits)) : nq;
    const std::uint64_t sx = wave_sum(v.x);                        // lanes 1..63: service x
    const std::uint64_t s0 = wave_sum(m ? umax64(ls, v.x) : 0ull);  // lane 0: max(sense, x)
    t.svc_sum += lane == 0 ? s0 : sx;
    const std::uint64_t seq0 = t.seq;  // sequence number of the batch's first record
    t.seq += 64 * nq;
    // Per-step totals of the 64 records, in closed form (lane k: step k).
    // Record j completes at done_j = max(pd_j, top - x (63 - j)), with pd_0 =
    // lead and pd_j = P for j >= 1 (P = lead with contention, else the issue
    // time).  The channel term grows with j, so among j = 1..63 the last cnt
    // records follow it and the others wait for P; the largest such record is
    // max(lead, top).
    if (m) {
        const std::uint64_t x = v.x;
        const std::uint64_t P = a.contention ? lead : q.issue;
        const std::uint64_t d0 = umax64(lead, top - 63 * x);
        std::uint64_t cnt = 0;  // records 1..63 on the channel side
        if (top >= P) {
            const std::uint64_t D = top - P;
            std::uint64_t tmax = 0;  // largest t <= 62 with x t <= D (x t <= 64 x <= top)
            for (std::uint64_t stp = 32; stp != 0; stp >>= 1) {
                if (tmax + stp <= 62 && x * (tmax + stp) <= D) {
                    tmax += stp;
                }
            }
            cnt = tmax + 1;
        }
        // sum_j done_j - 64 issue, exactly in 128 bits
        std::uint64_t lo = d0, hi = 0;
        const auto add = [&](std::uint64_t f, std::uint64_t w) {  // += f * w
            const std::uint64_t pl = f * w;
            const std::uint64_t ph = __umul64hi(f, w);
            const std::uint64_t n2 = lo + pl;
            hi += ph + (n2 < lo ? 1u : 0u);
            lo = n2;
        };
        const auto sub = [&](std::uint64_t f, std::uint64_t w) {  // -= f * w
            const std::uint64_t pl = f * w;
            const std::uint64_t ph = __umul64hi(f, w);
            hi -= ph + (lo < pl ? 1u : 0u);
            lo -= pl;
        };
        add(63 - cnt, P);
        add(cnt, top);
        sub(x, cnt * (cnt - (cnt != 0 ? 1 : 0)) / 2);
        sub(64, q.issue);
        const std::uint64_t n2 = t.lat_lo + lo;
        t.lat_hi += hi + (n2 < t.lat_lo ? 1u : 0u);
        t.lat_lo = n2;
        const std::uint64_t most = umax64(lead, top);
        t.mk = umax64(t.mk, most);
        t.lat_max = umax64(t.lat_max, most - q.issue);
    }
    // Completions.  Record j >= 1 of step k completes at max(P_k, top_k -
    // x_k (63 - j)) and record 0 at D0_k.  Lane j writes record j of every
    // step (whole 512-B rows: a row left partly written for a later store
    // costs more than the selects), taking P_k, top_k and D0_k from lane k by
    // shuffles; with one transfer time for the whole batch x (63 - j) is a
    // per-lane constant.  Nothing is outstanding here (the batch's values
    // were read above); saying so keeps a conservative wait for vector
    // memory out of the store loop, which would drain the stores.
    const std::uint64_t x0 = readlane64(v.x, 0);
    const bool xuni = __ballot(m && v.x != x0) == 0;
    const std::uint64_t back = static_cast<std::uint64_t>(63 - lane);
    const std::uint64_t P = a.contention ? lead : q.issue;
    const std::uint64_t D0 = umax64(lead, top - 63 * v.x);
    // Status bytes four steps at a time: 4 for a page-register hit (every
    // record but a sensing lane 0), 0 otherwise; with hybrid sampling, 8 more
    // for each record the sampler picks (record j of step k has sequence
    // number seq0 + 64 k + j and key (page, range, read), as in the general
    // path).  Lane l takes records 4 (l & 15) .. + 3 of step k + (l >> 4).
    // They are made next to the completion stores of the same four steps, so
    // that the sampler's hashes run while those stores drain.
    const bool stat = status != nullptr || a.hybrid;
    const bool words = status != nullptr && (reinterpret_cast<std::uintptr_t>(status) & 3u) == 0;
    const auto status4 = [&](int k) {
        const int ks = k + (lane >> 4);
        // every lane takes part in the shuffles
        const std::uint32_t kp = static_cast<std::uint32_t>(
            __shfl(static_cast<int>(q.page1), ks < q.n ? ks : 0));
        const std::uint32_t kr = static_cast<std::uint32_t>(
            __shfl(static_cast<int>(q.rid), ks < q.n ? ks : 0));
        if (ks < q.n) {
            const std::uint32_t r0 = 4u * static_cast<std::uint32_t>(lane & 15);
            const bool sense = r0 == 0 && ((hits >> ks) & 1u) == 0;
            std::uint32_t word = sense ? 0x04040400u : 0x04040404u;
            if (a.hybrid) {
                const std::uint64_t key =
                    ((static_cast<std::uint64_t>(kp) - 1) << a.page_shift) ^
                    (static_cast<std::uint64_t>(kr) << 32);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const std::uint64_t qn =
                        seq0 + static_cast<std::uint64_t>(ks) * kWave + r0 + u;
                    const bool sampled =
                        qn < a.hybrid_warmup ||
                        (a.hybrid_threshold != 0 && mix64(qn ^ key) <= a.hybrid_threshold);
                    if (sampled) {
                        word |= 8u << (8 * u);
                        ++t.n_hyb;
                    }
                }
            }
            if (status != nullptr) {
                std::uint8_t* out =
                    status + q.first + static_cast<std::size_t>(ks) * kWave + r0;
                if (words) {
                    *reinterpret_cast<std::uint32_t*>(out) = word;
                } else {
                    out[0] = static_cast<std::uint8_t>(word);
                    out[1] = static_cast<std::uint8_t>(word >> 8);
                    out[2] = static_cast<std::uint8_t>(word >> 16);
                    out[3] = static_cast<std::uint8_t>(word >> 24);
                }
            }
        }
    };
    std::uint64_t* out = completion + q.first + lane;
    wait_vector_loads();
    const bool z = lane == 0;
    if (xuni) {
        const std::uint64_t xm = x0 * back;
        int k = 0;
        for (; k + 4 <= q.n; k += 4) {
            std::uint64_t pk[4], tk[4], dk[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                pk[u] = shfl64(P, k + u);
                tk[u] = shfl64(top, k + u);
                dk[u] = shfl64(D0, k + u);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const std::uint64_t done = umax64(pk[u], tk[u] - xm);
                put_done(&out[static_cast<std::size_t>(k + u) * kWave], z ? dk[u] : done);
            }
            if (stat) {
                status4(k);
            }
        }
        const int kt = k;
        for (; k < q.n; ++k) {
            const std::uint64_t done = umax64(shfl64(P, k), shfl64(top, k) - xm);
            const std::uint64_t d = shfl64(D0, k);
            put_done(&out[static_cast<std::size_t>(k) * kWave], z ? d : done);
        }
        if (stat && kt < q.n) {
            status4(kt);
        }
    } else {
        for (int k = 0; k < q.n; ++k) {
            const std::uint64_t xm = shfl64(v.x, k) * back;
            const std::uint64_t done = umax64(shfl64(P, k), shfl64(top, k) - xm);
            const std::uint64_t d = shfl64(D0, k);
            put_done(&out[static_cast<std::size_t>(k) * kWave], z ? d : done);
        }
        if (stat) {
            for (int k = 0; k < q.n; k += 4) {
                status4(k);
            }
        }
    }
}

// fold_apply for a batch that holds split steps: lane r is run r, m records
// from lane lo of its step, all issued together and reading one page.  The
// run-level maps scan as in fold_apply with the channel moving m records;
// with e = lo + m - 1 the run's records complete at
//   record lo:           max(lead, top - x (m - 1))
//   record j > lo:       max(P, top - x (e - j))
// (P = lead with contention, else the issue time).  Rows are stored whole:
// lane j of a row takes the run its record belongs to, found by walking the
// runs row by row (a row's second run starts at a nonzero lane).
__device__ __forceinline__ void fold_apply_runs(const KArgs& a, const std::uint64_t* xp,
                                                const LinBatchT<true>& q, int lane,
                                                std::uint64_t* p_busy, std::uint64_t* c_busy,
                                                std::uint32_t* p_tag, std::uint64_t* completion,
                                                std::uint8_t* status, ApplySums& t,
                                                std::uint64_t* mt_p, std::uint64_t* mt_c)
{
    const StepView v = step_view(a, xp, q, lane);
    const bool m = v.m;
    const std::uint32_t pkey = m ? v.d.plane : 0u;
    const std::uint32_t ckey = m ? v.d.chan : 0u;
    const Group gp = group_plane_runs(a, q.page1, pkey, m, v.active, lane, mt_p);
    const Group gc = group_by(ckey, a.cbits, m, v.active, lane, mt_c);
    const std::uint32_t tag = m ? p_tag[pkey] : 0u;
    const std::uint64_t pbusy = m ? p_busy[pkey] : 0ull;
    const std::uint64_t cbusy = m ? c_busy[ckey] : 0ull;
    std::uint32_t prev1 = static_cast<std::uint32_t>(
        __shfl(static_cast<int>(q.page1), gp.pred < 0 ? lane : gp.pred));
    if (gp.pred < 0) {
        prev1 = tag;
    }
    const bool lhit = m && prev1 == q.page1;
    const std::uint64_t ls = lhit ? 0ull : a.read_ps;
    const std::uint64_t rm = m ? q.m : 1u;
    const std::uint64_t x = v.x;
    const std::uint64_t cx = rm * x;
    std::uint64_t Ap = 0, Bp = 0, Ac = 0, Bc = 0;
    if (m) {
        Ap = ls;
        Bp = q.issue + ls;
        Ac = cx;
        Bc = q.issue + cx;
    }
    if (a.contention) {
        scan_pair(gp, Ap, Bp, gc, Ac, Bc, v.d, m, v.active, ls, cx, lane);
    } else {
        scan_group(gc, Ac, Bc, lane);
    }
    const std::uint64_t lead = a.contention ? umax64(pbusy + Ap, Bp) : q.issue + ls;
    const std::uint64_t top = umax64(cbusy + Ac, Bc);
    if (m && lane == gp.last) {
        if (a.contention) {
            p_busy[pkey] = lead;
        }
        p_tag[pkey] = q.page1;
    }
    if (m && lane == gc.last) {
        c_busy[ckey] = top;
    }
    const std::uint64_t P = a.contention ? lead : q.issue;
    const std::uint64_t D0 = umax64(lead, top - (rm - 1) * x);
    // accounting: all modeled reads; every record after a run's first hits,
    // the first when its page was buffered
    const std::uint64_t recs = static_cast<std::uint64_t>(q.rows) * kWave;
    if (lane == 0) {
        t.n_rec += recs;
        t.n_mod += recs;
        t.n_rd += recs;
    }
    if (m) {
        t.n_hit += rm - 1 + (lhit ? 1u : 0u);
        t.svc_sum += umax64(ls, x) + (rm - 1) * x;
        // sum of the run's completions - m issue, exactly in 128 bits: among
        // records lo + 1 .. e the last cnt follow the channel, the others P
        std::uint64_t cnt = 0;
        if (rm >= 2 && top >= P) {
            const std::uint64_t D = top - P;
            std::uint64_t tmax = 0;  // largest t <= m - 2 with x t <= D
            for (std::uint64_t stp = 32; stp != 0; stp >>= 1) {
                if (tmax + stp <= rm - 2 && x * (tmax + stp) <= D) {
                    tmax += stp;
                }
            }
            cnt = tmax + 1;
        }
        std::uint64_t lo = D0, hi = 0;
        const auto add = [&](std::uint64_t f, std::uint64_t w) {  // += f * w
            const std::uint64_t pl = f * w;
            const std::uint64_t ph = __umul64hi(f, w);
            const std::uint64_t n2 = lo + pl;
            hi += ph + (n2 < lo ? 1u : 0u);
            lo = n2;
        };
        const auto sub = [&](std::uint64_t f, std::uint64_t w) {  // -= f * w
            const std::uint64_t pl = f * w;
            const std::uint64_t ph = __umul64hi(f, w);
            hi -= ph + (lo < pl ? 1u : 0u);
            lo -= pl;
        };
        add(rm - 1 - cnt, P);
        add(cnt, top);
        sub(x, cnt * (cnt - (cnt != 0 ? 1 : 0)) / 2);
        sub(rm, q.issue);
        const std::uint64_t n2 = t.lat_lo + lo;
        t.lat_hi += hi + (n2 < t.lat_lo ? 1u : 0u);
        t.lat_lo = n2;
        const std::uint64_t most = umax64(lead, top);
        t.mk = umax64(t.mk, most);
        t.lat_max = umax64(t.lat_max, most - q.issue);
    }
    const std::uint64_t seq0 = t.seq;
    t.seq += recs;
    const std::uint32_t e = m ? q.lo + q.m - 1 : 0u;
    const std::uint32_t hit1 = lhit ? 1u : 0u;
    wait_vector_loads();
    int ra = 0;  // the row's first run (wave-uniform)
    for (int r = 0; r < q.rows; ++r) {
        const bool two = ra + 1 < q.n && rl32(q.lo, ra + 1) != 0;
        const int rb = two ? ra + 1 : ra;
        const std::uint32_t kb = two ? rl32(q.lo, rb) : 0u;
        const bool second = two && static_cast<std::uint32_t>(lane) >= kb;
        const auto pick64 = [&](std::uint64_t val) {
            const std::uint64_t va = readlane64(val, ra);
            const std::uint64_t vb = readlane64(val, rb);
            return second ? vb : va;
        };
        const auto pick32 = [&](std::uint32_t val) {
            const std::uint32_t va = rl32(val, ra);
            const std::uint32_t vb = rl32(val, rb);
            return second ? vb : va;
        };
        const std::uint64_t rP = pick64(P);
        const std::uint64_t rtop = pick64(top);
        const std::uint64_t rD0 = pick64(D0);
        const std::uint64_t rx = pick64(x);
        const std::uint32_t re = pick32(e);
        const std::uint32_t j = static_cast<std::uint32_t>(lane);
        const bool first = j == (second ? kb : 0u);
        const std::uint64_t done =
            first ? rD0 : umax64(rP, rtop - rx * static_cast<std::uint64_t>(re - j));
        const std::size_t at = q.first + static_cast<std::size_t>(r) * kWave + lane;
        put_done(&completion[at], done);
        if (status != nullptr || a.hybrid) {
            std::uint8_t st = first && pick32(hit1) == 0 ? 0u : 4u;
            if (a.hybrid) {
                const std::uint64_t key =
                    ((static_cast<std::uint64_t>(pick32(q.page1)) - 1) << a.page_shift) ^
                    (static_cast<std::uint64_t>(pick32(q.rid)) << 32);
                const std::uint64_t qn = seq0 + static_cast<std::uint64_t>(r) * kWave + j;
                if (qn < a.hybrid_warmup ||
                    (a.hybrid_threshold != 0 && mix64(qn ^ key) <= a.hybrid_threshold)) {
                    st |= 8u;
                    ++t.n_hyb;
                }
            }
            if (status != nullptr) {
                status[at] = st;
            }
        }
        ra = rb + 1;
    }
}

// The apply pass copies a tile's step descriptors into LDS with its other
// set-up loads (tiles of up to kStageSteps steps, 4 KiB): read per window
// from memory instead, each read would wait for the previous window's
// completion stores, vector memory completing in issue order.
constexpr std::uint32_t kStageSteps = 256;

__host__ __device__ __forceinline__ std::uint32_t staged_steps(const KArgs& a)
{
    return a.tile <= kStageSteps * kWave ? a.tile / kWave : 0u;
}

// Byte offset of the staged descriptors in the apply pass's LDS (after the
// fences, plane busy, channel busy and plane tags; 16-byte aligned).
__host__ __device__ __forceinline__ std::size_t apply_desc_offset(const KArgs& a)
{
    return (8ull * (a.r_nfence + a.Rp + a.Rc) + 4ull * a.Rp + 15ull) & ~15ull;
}

// Byte offset of the apply pass's lane-matching tables (plane table, then
// channel table) after its state; 16-byte aligned.
__host__ __device__ __forceinline__ std::size_t apply_match_offset(const KArgs& a)
{
    return apply_desc_offset(a) + 16ull * staged_steps(a);
}

// Byte offset of the apply pass's stripe table (Rp words), after the
// lane-matching tables when the run keeps them.
__host__ __device__ __forceinline__ std::size_t apply_stripe_offset(const KArgs& a)
{
    return apply_match_offset(a) + (a.match_lds ? 8ull * (a.Rp + a.Rc) : 0ull);
}

// A tile's plane carry-ins are packed like its summaries: word w of the
// mask covers planes [64 w, 64 w + 64), so lane l reads bit l of each word.
// Eight words' carries are in flight before any is written.
__device__ __forceinline__ void load_plane_carry(const KArgs& a, const MaskWord* tmask,
                                                 const PlaneCarry* pcarry, std::size_t tile,
                                                 std::uint64_t* p_busy, std::uint32_t* p_tag,
                                                 int lane)
{
    constexpr int kWords = 8;
    const std::uint32_t words = mask_words(a);
    const MaskWord* tm = tmask + tile * words;
    const PlaneCarry* pc = pcarry + tile * a.Rp;
    const std::uint64_t below = lanemask_lt(lane);
    // (unrolled over the at most kMaxPlanes / 64 words: a loop back edge
    // would make the compiler wait for every carry load before the next)
#pragma unroll
    for (std::uint32_t w0 = 0; w0 < kMaxPlanes / kWave; w0 += kWords) {
        if (w0 >= words) {
            break;
        }
        // the mask words first, then the carries: vector loads complete in
        // issue order, so a word loaded after a carry would wait for it
        MaskWord mw[kWords];
#pragma unroll
        for (int k = 0; k < kWords; ++k) {
            mw[k] = w0 + k < words ? tm[w0 + k] : MaskWord{0, 0, 0};
        }
        PlaneCarry c[kWords];
        bool has[kWords];
#pragma unroll
        for (int k = 0; k < kWords; ++k) {
            has[k] = ((mw[k].bits >> lane) & 1ull) != 0;
            if (has[k]) {
                c[k] = pc[mw[k].base + static_cast<std::uint32_t>(__popcll(mw[k].bits & below))];
            }
        }
#pragma unroll
        for (int k = 0; k < kWords; ++k) {
            if (has[k]) {
                const std::uint32_t r = (w0 + k) * kWave + static_cast<std::uint32_t>(lane);
                p_busy[r] = c[k].busy;
                p_tag[r] = static_cast<std::uint32_t>(c[k].tag1);
            }
        }
    }
}

__device__ __forceinline__ void load_chan_carry(const KArgs& a, const std::uint64_t* ccarry,
                                                std::size_t tile, std::uint64_t* c_busy, int lane)
{
    constexpr int kPer = 4;
    const std::uint64_t* cc = ccarry + tile * a.Rc;
    for (std::uint32_t r0 = 0; r0 < a.Rc; r0 += kPer * kWave) {
        std::uint64_t v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const std::uint32_t r = r0 + k * kWave + static_cast<std::uint32_t>(lane);
            v[k] = r < a.Rc ? cc[r] : 0ull;
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const std::uint32_t r = r0 + k * kWave + static_cast<std::uint32_t>(lane);
            if (r < a.Rc) {
                c_busy[r] = v[k];
            }
        }
    }
}

// Runs of descriptor rows r0 .. r1 - 1 of a window (lane r holding row r's
// descriptor sd, its split side entry sp and range id; smask: the split
// rows) laid out one run per lane, at most 64: row r's first run sits at
// lane (r - r0) + the split rows in [r0, r), its second run after it.
__device__ __forceinline__ void expand_rows(LinBatchT<true>& q, const StepDesc& sd,
                                            const SplitDesc& sp,
                                            std::uint32_t rid, std::uint64_t smask, int r0,
                                            int r1, std::size_t w0, int lane)
{
    const std::uint64_t below0 = lanemask_lt(r0);
    const auto before = [&](int r) {  // runs of rows r0 .. r - 1
        return (r - r0) + __popcll(smask & lanemask_lt(r) & ~below0);
    };
    int r = r0;  // the last row whose first run is at or before this lane
    for (int stp = 32; stp != 0; stp >>= 1) {
        if (r + stp < r1 && before(r + stp) <= lane) {
            r += stp;
        }
    }
    const int nruns = before(r1 - 1) + 1 + static_cast<int>((smask >> (r1 - 1)) & 1ull);
    const bool second = lane > before(r);
    const bool two = ((smask >> r) & 1ull) != 0;
    const std::uint32_t p1 = static_cast<std::uint32_t>(__shfl(static_cast<int>(sd.page1), r));
    const std::uint32_t by = static_cast<std::uint32_t>(__shfl(static_cast<int>(sd.bytes), r));
    const std::uint64_t is = shfl64(sd.issue, r);
    const std::uint32_t ra = static_cast<std::uint32_t>(__shfl(static_cast<int>(rid), r));
    const std::uint32_t pb = static_cast<std::uint32_t>(__shfl(static_cast<int>(sp.page1b), r));
    const std::uint32_t k = static_cast<std::uint32_t>(__shfl(static_cast<int>(sp.k), r));
    const std::uint32_t rb = static_cast<std::uint32_t>(__shfl(static_cast<int>(sp.ridb), r));
    const bool in = lane < nruns;
    q.page1 = in ? (second ? pb : p1) : 0u;
    q.bytes = by & ~kSplitFlag;
    q.issue = is;
    q.rid = second ? rb : ra;
    q.m = two ? (second ? kWave - k : k) : kWave;
    q.lo = second ? k : 0u;
    q.first = w0 + static_cast<std::size_t>(r0) * kWave;
    q.n = nruns;
    q.rows = r1 - r0;
    q.split = (smask & lanemask_lt(r1) & ~below0) != 0;
}

// Folds the apply pass's pending batch (fold_apply_runs when it holds a
// split step; kGiven: page-register hits from `hits`) and empties it.
template <bool kR, bool kGiven>
__device__ __forceinline__ void fold_batch(const KArgs& a, const std::uint64_t* xp,
                                           LinBatchT<kR>& q, int lane, std::uint64_t* p_busy,
                                           std::uint64_t* c_busy, std::uint32_t* p_tag,
                                           std::uint64_t* completion, std::uint8_t* status,
                                           ApplySums& t, std::uint64_t* mt_p, std::uint64_t* mt_c,
                                           const std::uint8_t* hits)
{
    if constexpr (kR) {
        if (q.any_split()) {
            fold_apply_runs(a, xp, q, lane, p_busy, c_busy, p_tag, completion, status, t, mt_p,
                            mt_c);
            q.clear();
            return;
        }
    }
    fold_apply<kR, kGiven>(a, xp, q, lane, p_busy, c_busy, p_tag, completion, status, t, mt_p,
                           mt_c, hits);
    q.clear();
}

// The apply pass over one tile.  kSplit: the tile holds split steps (packed
// records; the summary pass says so per tile), which its batches take as
// runs; without it the body is the whole-step one, whose folds and stores
// then keep every register the pass has (the split-capable body needs more:
// compiled into the same code path it would make the whole-step folds spill).
template <bool kRefresh, bool kHits, bool kStaged, bool kPacked, bool kSplit, bool kWide = false>
__device__ __forceinline__ void apply_tile(
    const KArgs& a, const void* rec, std::size_t n, std::uint64_t base_ps,
    const PlaneCarry* pcarry, const MaskWord* tmask, const std::uint64_t* ccarry,
    const std::uint64_t* tile_seq, std::uint64_t* completion, std::uint8_t* status,
    DevReport* tile_rep, const std::uint8_t* hits, const StepDesc* desc, std::uint64_t* sm,
    std::uint64_t* xp)
{
    std::uint64_t* fence = sm;
    std::uint64_t* p_busy = fence + a.r_nfence;
    std::uint64_t* c_busy = p_busy + a.Rp;
    std::uint32_t* p_tag = reinterpret_cast<std::uint32_t*>(c_busy + a.Rc);
    const int lane = threadIdx.x;
    const std::size_t tile = blockIdx.x;
    // set-up loads in flight together: the fences, then the carry-ins, which
    // exist for the planes the tile touches (the only ones it reads)
    const std::size_t begin = tile * a.tile;
    const std::size_t end = begin + a.tile < n ? begin + a.tile : n;
    // kStaged: the launch found descriptors and a tile of at most kStageSteps
    // steps (a template parameter: as a run-time flag it costs registers)
    constexpr bool stage = kStaged;
    StepDesc* sdesc = reinterpret_cast<StepDesc*>(reinterpret_cast<unsigned char*>(sm) +
                                                  apply_desc_offset(a));
    std::uint64_t* mt_p = a.match_lds ? reinterpret_cast<std::uint64_t*>(
                                            reinterpret_cast<unsigned char*>(sm) +
                                            apply_match_offset(a))
                                      : nullptr;
    std::uint64_t* mt_c = a.match_lds ? mt_p + a.Rp : nullptr;
    const std::size_t tsteps = (end - begin + kWave - 1) / kWave;
    const FenceRegs fr = fetch_fences(a, lane);
    const std::uint64_t xv = fetch_xfer(a, lane);
    constexpr int kDescPerLane = static_cast<int>(kStageSteps) / kWave;
    StepDesc dv[kDescPerLane];
#pragma unroll
    for (int k = 0; k < kDescPerLane; ++k) {
        const std::size_t j = static_cast<std::size_t>(k * kWave + lane);
        dv[k] = StepDesc{0, 0, 0};
        if (stage && j < tsteps) {
            dv[k] = desc[begin / kWave + j];
        }
    }
    load_plane_carry(a, tmask, pcarry, tile, p_busy, p_tag, lane);
    load_chan_carry(a, ccarry, tile, c_busy, lane);
    store_fences(a, fr, fence, lane);
    store_xfer(xp, xv, lane);
    if (a.match_lds) {
        for (std::uint32_t r = lane; r < a.Rp + a.Rc; r += kWave) {
            mt_p[r] = 0;
        }
    }
    std::uint32_t* stab = nullptr;
    if (a.stripe_lds) {
        stab = reinterpret_cast<std::uint32_t*>(reinterpret_cast<unsigned char*>(sm) +
                                                apply_stripe_offset(a));
        fill_stripe_table(a, stab, lane);
    }
    if (stage) {
#pragma unroll
        for (int k = 0; k < kDescPerLane; ++k) {
            const std::size_t j = static_cast<std::size_t>(k * kWave + lane);
            if (j < tsteps) {
                sdesc[j] = dv[k];
            }
        }
    }
    __syncthreads();
    // the batch folds' accumulators, and the ones only the general path adds to
    ApplySums t{0, 0, 0, 0, 0, 0, 0, 0, 0, tile_seq[tile], 0};
    std::uint64_t n_byp = 0, n_uns = 0, n_wr = 0, n_prog = 0;
    RangeCache rc = empty_cache();
    RangeCache rcu = empty_cache();  // wave-uniform copy for linear steps
    LinBatchT<kSplit> q = empty_batch<kSplit>();
    constexpr int kFull = kSplit ? kWave - 1 : kWave;  // room for a split step's runs
    std::uint32_t lin_miss = 0;  // steps in a row that were not linear (wave-uniform)
    // Windows of 64 steps.  A window whose steps the summary pass found all
    // linear is replayed from their descriptors alone, without reading its
    // records; any other window streams its records through the pipeline.
    for (std::size_t w0 = begin; w0 < end; w0 += kWave * kWave) {
        const std::size_t wend = w0 + kWave * kWave < end ? w0 + kWave * kWave : end;
        if (desc != nullptr) {
            const int nst = static_cast<int>((wend - w0 + kWave - 1) / kWave);
            StepDesc sd{0, 0, 0};
            if (lane < nst) {
                if (stage) {
                    sd = sdesc[(w0 - begin) / kWave + lane];
                } else {
                    sd = desc[w0 / kWave + lane];
                }
            }
            const std::uint64_t all = nst == kWave ? ~0ull : ((1ull << nst) - 1);
            // (a split step's descriptor in a tile not marked split: the
            // window is streamed, where such a step takes the general path)
            const bool ok = sd.bytes != 0 && (kSplit || (sd.bytes & kSplitFlag) == 0);
            if (__ballot(lane < nst && ok) == all) {
                const std::uint32_t rid =
                    a.desc_rid != nullptr && lane < nst ? a.desc_rid[w0 / kWave + lane] : 0u;
                const std::uint64_t smask =
                    kSplit ? __ballot(lane < nst && (sd.bytes & kSplitFlag) != 0) : 0ull;
                // split steps have their second runs in the side array; the
                // window's runs fold in one batch, or in two when they exceed 64
                SplitDesc sp{0, 0, 0, 0};
                if (kSplit && ((smask >> lane) & 1ull) != 0) {
                    sp = a.desc_split[w0 / kWave + lane];
                }
                if constexpr (!kSplit) {
                    q.page1 = sd.page1;
                    q.bytes = sd.bytes;
                    q.issue = sd.issue;
                    q.rid = rid;
                    q.first = w0;
                    q.n = nst;
                    q.rows = nst;
                    fold_batch<kSplit, kHits>(a, xp, q, lane, p_busy, c_busy, p_tag, completion,
                               status, t, mt_p, mt_c, hits);
                } else {
                    const int runs = nst + __popcll(smask);
                    const int half = runs <= kWave ? nst : nst / 2;
                    for (int r0 = 0; r0 < nst;) {
                        const int r1 = r0 == 0 ? half : nst;
                        if (smask != 0) {
                            expand_rows(q, sd, sp, rid, smask, r0, r1, w0, lane);
                        } else {
                            q.page1 = sd.page1;
                            q.bytes = sd.bytes;
                            q.issue = sd.issue;
                            q.rid = rid;
                            q.m = kWave;
                            q.lo = 0;
                            q.first = w0;
                            q.n = nst;
                            q.rows = nst;
                        }
                        fold_batch<kSplit, kHits>(a, xp, q, lane, p_busy, c_busy, p_tag, completion,
                                   status, t, mt_p, mt_c, hits);
                        r0 = r1;
                    }
                }
                continue;
            }
        }
        // (the four-wave form keeps two steps in flight)
        constexpr int kDepth = kPacked && kWide ? 2 : kPipe;
        constexpr std::size_t kSpan = static_cast<std::size_t>(kDepth) * kWave;
        using Pipe = std::conditional_t<kPacked, PackedPipeT<kDepth>, RecordPipe>;
        static_assert(kPacked || kDepth == kPipe, "32-byte records keep kPipe steps");
        Pipe pipe;
        pipe.issue(rec, w0, wend, lane);
        for (std::size_t g = w0; g < wend; g += kSpan) {
            pipe.advance(rec, g + kSpan, wend, lane);
            const std::size_t gend = g + kSpan < wend ? g + kSpan : wend;
            for (std::size_t s = g; s < gend; s += kWave) {
                typename Pipe::Step sr;
                pipe.take(sr);
                const std::size_t i = s + lane;
                const bool valid = i < end;
                if ((kHits || a.slots == 1) && a.lead == nullptr) {
                    // batched as in the summary pass
                    LinStep ls;
                    bool lin = false;
                    if (lin_miss < kLinGiveUp || (s / kWave) % kLinProbe == 0) {
                        lin = detect_step<kRefresh, kSplit>(a, fence, rcu, sr, base_ps,
                                                            s + kWave <= end, lane, ls);
                        lin_miss = lin ? 0u : lin_miss + 1u;
                    }
                    if (lin) {
                        if (ls.k == 0) {
                            q.push(ls.page1, ls.issue, ls.bytes, s, ls.rid);
                        } else {
                            q.push_split(ls.page1, ls.page1b, ls.k, ls.issue, ls.bytes, s,
                                         ls.rid, ls.ridb);
                        }
                    }
                    if (q.n != 0 && (!lin || q.n >= kFull || s + kWave >= wend)) {
                        fold_batch<kSplit, kHits>(a, xp, q, lane, p_busy, c_busy, p_tag, completion,
                               status, t, mt_p, mt_c, hits);
                    }
                    if (lin) {
                        continue;
                    }
                }
                uint4 x, y;
                step_records(sr, lane, x, y);
                Dec d = valid ? decode<kRefresh>(a, fence, rc, x, y, base_ps, stab)
                              : invalid_dec();
                if (!kPacked && a.lead != nullptr && valid && a.lead[i] != 0) {
                    d.cls = kClsFollower;  // timed by k_follow from its group's request
                }
                const bool m = valid && d.cls == kClsModeled;
                const bool hbit = kHits && valid && hits[i] != 0;
                const std::uint64_t active = __ballot(m);
                std::uint8_t st = static_cast<std::uint8_t>(d.cls);
                std::uint64_t done = 0;
                if (!kHits && active != 0 && run_step(a, d, active, lane)) {
                    const std::uint64_t xfer = lane_xfer(a, xp, d, m, active);
                    const std::uint64_t W = run_channel_max(d, xfer, lane);
                    const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
                    const std::uint32_t pkey = d.plane;
                    const std::uint32_t ckey = d.chan;
                    const std::uint32_t tag = p_tag[pkey];
                    const std::uint64_t pbusy = p_busy[pkey];
                    const std::uint64_t cbusy = c_busy[ckey];
                    const std::uint64_t i0 = readlane64(d.issue, 0);
                    const bool lhit = tag == page1;
                    const std::uint64_t ls = lhit ? 0ull : a.read_ps;
                    const std::uint64_t lead = a.contention ? umax64(pbusy, i0) + ls : i0 + ls;
                    std::uint64_t pd;
                    if (lane == 0) {
                        pd = lead;
                    } else {
                        pd = a.contention ? umax64(lead, d.issue) : d.issue;
                    }
                    const std::uint64_t k1 = static_cast<std::uint64_t>(lane + 1);
                    const std::uint64_t back = static_cast<std::uint64_t>(62 - lane);
                    const std::uint64_t cd =
                        umax64(cbusy + xfer * k1, lane == 63 ? W + xfer : W - xfer * back);
                    if (lane == 63) {
                        if (a.contention) {
                            p_busy[pkey] = pd;
                        }
                        p_tag[pkey] = page1;
                        c_busy[ckey] = cd;
                    }
                    done = umax64(pd, cd);
                    const bool hit = lane == 0 ? lhit : true;
                    const std::uint64_t svc = lane == 0 ? ls : 0ull;
                    if (a.hybrid) {
                        const std::uint64_t qn = t.seq + static_cast<std::uint64_t>(lane);
                        const std::uint64_t key = ((d.page1 - 1) << a.page_shift) ^
                                                  (static_cast<std::uint64_t>(d.range_id) << 32);
                        if (qn < a.hybrid_warmup ||
                            (a.hybrid_threshold != 0 && mix64(qn ^ key) <= a.hybrid_threshold)) {
                            st |= 8u;
                            ++t.n_hyb;
                        }
                    }
                    ++t.n_mod;
                    ++t.n_rd;
                    if (hit) {
                        st |= 4u;
                        ++t.n_hit;
                    }
                    t.mk = umax64(t.mk, done);
                    const std::uint64_t lat = done - d.issue;
                    add128(t.lat_lo, t.lat_hi, lat);
                    t.lat_max = umax64(t.lat_max, lat);
                    t.svc_sum += umax64(svc, xfer);
                    t.seq += 64;
                } else if (active != 0) {
                    const std::uint64_t xfer = lane_xfer(a, xp, d, m, active);
                    const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
                    const std::uint32_t pkey = m ? d.plane : 0u;
                    const std::uint32_t ckey = m ? d.chan : 0u;
                    const Group gp = group_by(pkey, a.pbits, m, active, lane, mt_p);
                    const Group gc = group_by(ckey, a.cbits, m, active, lane, mt_c);
                    // state reads come before this step's writes
                    const std::uint32_t tag = m ? p_tag[pkey] : 0u;
                    const std::uint64_t pbusy = m ? p_busy[pkey] : 0ull;
                    const std::uint64_t cbusy = m ? c_busy[ckey] : 0ull;
                    std::uint32_t prev1 = static_cast<std::uint32_t>(
                        __shfl(static_cast<int>(page1), gp.pred < 0 ? lane : gp.pred));
                    if (gp.pred < 0) {
                        prev1 = tag;
                    }
                    const bool hit = kHits ? (m && hbit) : (a.slots != 0 && m && prev1 == page1);
                    const std::uint64_t svc = plane_service(a, d.bits, hit);
                    std::uint64_t Ap = m ? svc : 0ull;
                    std::uint64_t Bp = m ? d.issue + svc : 0ull;
                    std::uint64_t Ac = m ? xfer : 0ull;
                    std::uint64_t Bc = m ? d.issue + xfer : 0ull;
                    if (a.contention) {
                        scan_pair(gp, Ap, Bp, gc, Ac, Bc, d, m, active, svc, xfer, lane);
                    } else {
                        scan_group(gc, Ac, Bc, lane);
                    }
                    const std::uint64_t pd =
                        a.contention ? (m ? umax64(pbusy + Ap, Bp) : 0ull) : d.issue + svc;
                    const std::uint64_t cd = m ? umax64(cbusy + Ac, Bc) : 0ull;
                    if (m && lane == gp.last) {
                        if (a.contention) {
                            p_busy[pkey] = pd;
                        }
                        p_tag[pkey] = page1;
                    }
                    if (m && lane == gc.last) {
                        c_busy[ckey] = cd;
                    }
                    if (m) {
                        done = umax64(pd, cd);
                        const std::uint64_t rank = __popcll(active & lanemask_lt(lane));
                        const std::uint64_t qn = t.seq + rank;
                        if (a.hybrid) {
                            const std::uint64_t key =
                                ((d.page1 - 1) << a.page_shift) ^
                                (static_cast<std::uint64_t>(d.range_id) << 32) ^ dec_op(d.bits);
                            const bool sampled =
                                qn < a.hybrid_warmup ||
                                (a.hybrid_threshold != 0 && mix64(qn ^ key) <= a.hybrid_threshold);
                            if (sampled) {
                                st |= 8u;
                                ++t.n_hyb;
                            }
                        }
                        ++t.n_mod;
                        if ((d.bits & 1u) == 0) {
                            ++t.n_rd;
                            if (hit) {
                                st |= 4u;
                                ++t.n_hit;
                            }
                        } else {
                            n_wr += (d.bits & 4u) ? 0u : 1u;
                            if (svc != 0) {
                                st |= 16u;
                                ++n_prog;
                            }
                        }
                        t.mk = umax64(t.mk, done);
                        const std::uint64_t lat = done - d.issue;
                        add128(t.lat_lo, t.lat_hi, lat);
                        t.lat_max = umax64(t.lat_max, lat);
                        t.svc_sum += umax64(svc, xfer);
                    }
                    t.seq += __popcll(active);
                }
                if (valid) {
                    ++t.n_rec;
                    if (d.cls == kClsBypass) {
                        done = d.issue;
                        ++n_byp;
                    } else if (d.cls == kClsUnsupported) {
                        done = ~0ull;
                        ++n_uns;
                    }
                    put_done(&completion[i], done);
                    if (status != nullptr) {
                        status[i] = st;
                    }
                }
            }
        }
    }
    // 128-bit latency sum: reduce the high words, then the low words with
    // their carries.
    std::uint64_t hi = wave_sum(t.lat_hi);
    std::uint64_t carry = 0;
    std::uint64_t v = t.lat_lo;
    for (int o = 32; o > 0; o >>= 1) {
        const std::uint64_t other = shfl64(v, threadIdx.x ^ o);
        const std::uint64_t oc = shfl64(carry, threadIdx.x ^ o);
        const std::uint64_t sum = v + other;
        carry = carry + oc + (sum < v ? 1u : 0u);
        v = sum;
    }
    hi += carry;
    const std::uint64_t vals[14] = {
        wave_sum(t.n_rec), wave_sum(t.n_mod), wave_sum(n_byp), wave_sum(n_uns), wave_sum(t.n_rd),
        wave_sum(n_wr),  wave_sum(t.n_hit), wave_sum(n_prog), wave_sum(t.n_hyb), wave_max(t.mk),
        v,               hi,              wave_max(t.lat_max), wave_sum(t.svc_sum)};
    if (lane < 14) {
        unsigned long long out = 0;
#pragma unroll
        for (int k = 0; k < 14; ++k) {
            out = lane == k ? vals[k] : out;
        }
        tile_rep[tile].v[lane] = out;
    }
}

// Packed records: three waves per SIMD (at most 168 registers), since the
// general steps' chains of ballots, shuffles and LDS updates need the
// latency hiding and the streamed linear steps lose nothing.  32-byte
// records hold twice the bytes per step in registers and would spill.
// kWide: four waves per SIMD with two steps in flight, for large streams of
// general steps (k_apply 4.15 -> 3.59 ms at 2^28 random records); on streams
// of linear steps its spilled registers cost 7-15% of the pass.
template <bool kRefresh, bool kHits, bool kStaged = false, bool kPacked = false,
          bool kWide = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kWide ? 4 : (kPacked ? 3 : 1)))) void k_apply(
    KArgs a, const void* rec, std::size_t n, std::uint64_t base_ps, const PlaneCarry* pcarry,
    const MaskWord* tmask, const std::uint64_t* ccarry, const std::uint64_t* tile_seq,
    std::uint64_t* completion, std::uint8_t* status, DevReport* tile_rep,
    const std::uint8_t* hits, const StepDesc* desc)
{
    extern __shared__ std::uint64_t sm[];
    __shared__ std::uint64_t xp[33];
    if constexpr (kPacked) {
        if (a.tile_split != nullptr && a.tile_split[blockIdx.x] != 0) {
            apply_tile<kRefresh, kHits, kStaged, kPacked, true, kWide>(
                a, rec, n, base_ps, pcarry, tmask, ccarry, tile_seq, completion, status, tile_rep,
                hits, desc, sm, xp);
            return;
        }
    }
    apply_tile<kRefresh, kHits, kStaged, kPacked, false, kWide>(a, rec, n, base_ps, pcarry, tmask,
                                                                ccarry, tile_seq, completion,
                                                                status, tile_rep, hits, desc, sm,
                                                                xp);
}

// Folds the per-tile report partials into one report (sums, maxima and the
// 128-bit latency sum).  One block.
// Report reduction in two launches: blocks fold runs of tile reports into
// partials, then one block folds the partials.  A block's 256 threads are 16
// streams x 16 words (the 14 report words, the carry out of the 128-bit
// latency sum, padding); sums and maxima are exact in any order.
constexpr int kRepWords = 16;
constexpr int kRepCarry = 14;
constexpr int kRepParts = 256;

__device__ __forceinline__ void rep_join(int f, std::uint64_t& acc, std::uint64_t& carry,
                                         std::uint64_t v, std::uint64_t vcarry)
{
    if (f == R_MAKESPAN || f == R_LAT_MAX) {
        acc = umax64(acc, v);
    } else if (f == R_LAT_LO) {
        const std::uint64_t s2 = acc + v;
        carry += vcarry + (s2 < acc ? 1u : 0u);
        acc = s2;
    } else {
        acc += v;
    }
}

// in: `count` entries of kIn words (14: tile reports, kRepWords: partials);
// block b folds entries [b * per, (b + 1) * per).  With kFinal the single
// block writes the report (carry added into the high latency word), else a
// kRepWords partial per block.
template <int kIn, bool kFinal>
__global__ __launch_bounds__(256) void k_report(const std::uint64_t* in, std::size_t count,
                                                std::size_t per, std::uint64_t* out,
                                                std::uint32_t* disorder)
{
    __shared__ std::uint64_t acc_sh[16][kRepWords];
    __shared__ std::uint64_t carry_sh[16];
    const int t = threadIdx.x;
    const int f = t % kRepWords;
    const int stream = t / kRepWords;
    const std::size_t lo = static_cast<std::size_t>(blockIdx.x) * per;
    const std::size_t hi = lo + per < count ? lo + per : count;
    std::uint64_t acc = 0, carry = 0;
    // kBatch entries per stream are loaded before any is joined (one memory
    // round trip per batch, not per entry); entries past `hi` read as 0,
    // which every field's join leaves unchanged
    constexpr int kBatch = 8;
    for (std::size_t i0 = lo + stream; i0 < hi; i0 += 16 * kBatch) {
        std::uint64_t v[kBatch], vc[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const std::size_t i = i0 + 16 * static_cast<std::size_t>(k);
            v[k] = i < hi && f < kIn ? in[i * kIn + f] : 0ull;
            // a partial's carry word travels with its latency word
            vc[k] = i < hi && kIn == kRepWords && f == R_LAT_LO ? in[i * kIn + kRepCarry] : 0ull;
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            rep_join(f, acc, carry, f == kRepCarry ? 0ull : v[k], vc[k]);
        }
    }
    acc_sh[stream][f] = acc;
    if (f == R_LAT_LO) {
        carry_sh[stream] = carry;
    }
    __syncthreads();
    for (int half = 8; half > 0; half >>= 1) {
        if (stream < half) {
            std::uint64_t a0 = acc_sh[stream][f];
            std::uint64_t c0 = f == R_LAT_LO ? carry_sh[stream] : 0ull;
            rep_join(f, a0, c0, acc_sh[stream + half][f],
                     f == R_LAT_LO ? carry_sh[stream + half] : 0ull);
            acc_sh[stream][f] = a0;
            if (f == R_LAT_LO) {
                carry_sh[stream] = c0;
            }
        }
        __syncthreads();
    }
    if (stream == 0) {
        if (kFinal) {
            if (f < 14) {
                out[f] = f == R_LAT_HI ? acc_sh[0][f] + carry_sh[0] : acc_sh[0][f];
            } else if (f == 14) {
                // the run's disorder flag travels with the report, and is
                // cleared for the next run
                out[14] = disorder != nullptr ? *disorder : 0u;
                if (disorder != nullptr) {
                    *disorder = 0u;
                }
            }
        } else {
            out[static_cast<std::size_t>(blockIdx.x) * kRepWords + f] =
                f == kRepCarry ? carry_sh[0] : acc_sh[0][f];
        }
    }
}

// Folds `ntiles` tile reports into `rep` (parts: kRepParts * kRepWords words).
// ---- warp grouping (hbf_device.cu:1223-1231) ----------------------------
//
// The lanes of one warp instruction are consecutive records with one nonzero
// group id (flags bits 32-63); among them, modeled records with the same
// (range, media page) share the media request of the first.  k_lead marks
// every other such record with how far back that first record is; the
// summary and apply passes then time only the requests, and k_follow gives
// each marked record its request's completion.

constexpr std::size_t kLeadSpan = 1024;  // records per wave of k_lead
constexpr unsigned kFollowBlocks = 8192;

// One wave per kLeadSpan records; the 64 records before them are decoded
// too, as history.  Two windows of 64 records live in LDS: record i in slot
// ((i >> 6) & 1) * 64 + (i & 63).  A group of more than 64 records or with
// two issue times sets *err (the run is refused before anything is timed).
__global__ __launch_bounds__(64) void k_lead(KArgs a, const hbf_record32* rec, std::size_t n,
                                             std::uint8_t* lead, std::uint32_t* err)
{
    extern __shared__ std::uint64_t sm[];
    std::uint64_t* fence = sm;
    __shared__ std::uint64_t s_issue[2 * kWave];
    __shared__ std::uint64_t s_page1[2 * kWave];  // media page + 1; 0: not modeled
    __shared__ std::uint32_t s_group[2 * kWave];
    __shared__ std::uint32_t s_range[2 * kWave];
    const int lane = threadIdx.x;
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kLeadSpan;
    const std::size_t end = begin + kLeadSpan < n ? begin + kLeadSpan : n;
    load_fences(a, fence, lane);
    __syncthreads();
    RangeCache rc = empty_cache();
    std::uint32_t bad = 0;
    for (std::size_t s = begin >= kWave ? begin - kWave : begin; s < end; s += kWave) {
        const std::size_t i = s + lane;
        const int slot = static_cast<int>(((i >> 6) & 1u) * kWave + (i & 63u));
        std::uint32_t g = 0, rid = 0;
        std::uint64_t issue = 0, page1 = 0;
        if (i < end) {
            uint4 x, y;
            load_record(rec, i, x, y);
            g = y.w;
            issue = y.x | (static_cast<std::uint64_t>(y.y) << 32);
            if (g != 0) {
                const Dec d = decode<false>(a, fence, rc, x, y, 0);
                if (d.cls == kClsModeled) {
                    page1 = d.page1;
                    rid = d.range_id;
                }
            }
        }
        s_group[slot] = g;
        s_issue[slot] = issue;
        s_page1[slot] = page1;
        s_range[slot] = rid;
        __syncthreads();
        if (s >= begin && i < end) {
            std::uint32_t back = 0;
            if (g != 0) {
                // the group's earlier records: at most 63, all in the two windows
                for (std::size_t t = 1; t <= kWave && t <= i; ++t) {
                    const std::size_t j = i - t;
                    const int sj = static_cast<int>(((j >> 6) & 1u) * kWave + (j & 63u));
                    if (s_group[sj] != g) {
                        break;
                    }
                    if (t == kWave || s_issue[sj] != issue) {
                        bad = 1;
                        break;
                    }
                    if (page1 != 0 && s_page1[sj] == page1 && s_range[sj] == rid) {
                        back = static_cast<std::uint32_t>(t);
                    }
                }
            }
            lead[i] = static_cast<std::uint8_t>(back);
        }
        __syncthreads();
    }
    if (__ballot(bad != 0) != 0 && lane == 0) {
        atomicMax(err, 1u);
    }
}

// Each marked record takes its request's completion (final once k_apply
// has run: a request is never itself marked) and status kStGrouped, and is
// counted into frep: records that joined, reads, writes, makespan, latency
// sum (low, high words), latency maximum.
__global__ __launch_bounds__(256) void k_follow(const hbf_record32* rec, std::size_t n,
                                                std::uint64_t base_ps, const std::uint8_t* lead,
                                                std::uint64_t* comp, std::uint8_t* status,
                                                unsigned long long* frep)
{
    std::uint64_t cnt = 0, rd = 0, wr = 0, mk = 0, lo = 0, hi = 0, mx = 0;
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        const std::uint32_t back = lead[i];
        if (back == 0) {
            continue;
        }
        const std::uint64_t done = comp[i - back];
        comp[i] = done;
        if (status != nullptr) {
            status[i] = kStGrouped;
        }
        const uint4 y = reinterpret_cast<const uint4*>(rec + i)[1];
        const std::uint64_t issue = base_ps + (y.x | (static_cast<std::uint64_t>(y.y) << 32));
        const std::uint32_t op = y.z & 0xffu;
        ++cnt;
        rd += op == 0 ? 1u : 0u;
        wr += op == 1 ? 1u : 0u;
        mk = umax64(mk, done);
        const std::uint64_t lat = done - issue;
        const std::uint64_t l2 = lo + lat;
        hi += l2 < lo ? 1u : 0u;
        lo = l2;
        mx = umax64(mx, lat);
    }
    const std::uint64_t total = wave_sum(cnt);
    if (total == 0) {
        return;  // wave-uniform
    }
    // 128-bit latency sum across the wave: high words, then low words with
    // their carries
    hi = wave_sum(hi);
    std::uint64_t carry = 0;
    for (int o = 32; o > 0; o >>= 1) {
        const std::uint64_t other = shfl64(lo, threadIdx.x ^ o);
        const std::uint64_t oc = shfl64(carry, threadIdx.x ^ o);
        const std::uint64_t sum = lo + other;
        carry = carry + oc + (sum < lo ? 1u : 0u);
        lo = sum;
    }
    hi += carry;
    rd = wave_sum(rd);
    wr = wave_sum(wr);
    mk = wave_max(mk);
    mx = wave_max(mx);
    if ((threadIdx.x & 63u) == 0) {
        atomicAdd(&frep[0], static_cast<unsigned long long>(total));
        atomicAdd(&frep[1], static_cast<unsigned long long>(rd));
        atomicAdd(&frep[2], static_cast<unsigned long long>(wr));
        atomicMax(&frep[3], static_cast<unsigned long long>(mk));
        const unsigned long long old = atomicAdd(&frep[4], static_cast<unsigned long long>(lo));
        hi += old + lo < old ? 1u : 0u;
        atomicAdd(&frep[5], static_cast<unsigned long long>(hi));
        atomicMax(&frep[6], static_cast<unsigned long long>(mx));
    }
}

// The report's word 14 receives *disorder, which is then cleared (both skipped
// when disorder is null); `rep` holds two DevReports.
void launch_report(hipStream_t stream, const DevReport* tile_rep, std::size_t ntiles,
                   DevReport* rep, std::uint64_t* parts, std::uint32_t* disorder)
{
    const std::size_t per = (ntiles + kRepParts - 1) / kRepParts;
    const std::size_t nparts = per == 0 ? 0 : (ntiles + per - 1) / per;
    if (nparts == 0) {
        hipLaunchKernelGGL((k_report<kRepWords, true>), dim3(1), dim3(256), 0, stream, parts,
                           std::size_t{0}, std::size_t{1}, reinterpret_cast<std::uint64_t*>(rep),
                           disorder);
        return;
    }
    hipLaunchKernelGGL((k_report<14, false>), dim3(static_cast<unsigned>(nparts)), dim3(256), 0,
                       stream, reinterpret_cast<const std::uint64_t*>(tile_rep), ntiles, per,
                       parts, static_cast<std::uint32_t*>(nullptr));
    hipLaunchKernelGGL((k_report<kRepWords, true>), dim3(1), dim3(256), 0, stream, parts, nparts,
                       nparts, reinterpret_cast<std::uint64_t*>(rep), disorder);
}

}  // namespace

// ------------------------------------------------------------------------
// Scratch of the entry point that allocates nothing
// (hbfsim_amd_run_device_packed_noalloc): one array per device, part of the
// code object, so the entry point never calls an allocator.  Host code uses
// only the device address hipGetSymbolAddress returns for it (kept per device
// in noalloc_scratch below), never the array's name.  Every call on a device
// shares it; calls that overlap on one device race.  Nothing in it needs to
// start at zero: each kernel of a run writes every scratch word it reads
// before reading it, as with the engine's own reused scratch.

}  // namespace hbfamd

static __device__ __align__(256) unsigned char scratch[hbfamd::kNoAllocScratchBytes];

namespace hbfamd {

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};

// Looks the array's device address up once per device; `device` must be
// current.  Returns nullptr when the lookup fails.
void* noalloc_scratch(int device)
{
    if (device < 0 || device >= kMaxDevices) {
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[device] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess) {
            g_noalloc_ptr[device] = ptr;
        }
    }
    return g_noalloc_ptr[device];
}

}  // namespace

// ------------------------------------------------------------------------
// host side

struct engine {
    engine_config cfg;
    int device{0};
    KArgs args{};
    // ranges
    std::vector<range_rec> ranges;
    bool ranges_dirty{true};
    std::uint64_t* d_r_base{nullptr};
    std::uint64_t* d_r_length{nullptr};
    std::uint64_t* d_r_offset{nullptr};
    std::uint32_t* d_r_meta{nullptr};
    std::uint32_t* d_r_id{nullptr};
    std::size_t range_cap{0};
    // persistent state
    std::uint64_t* d_pbusy{nullptr};
    std::uint64_t* d_ptag{nullptr};
    std::uint64_t* d_cbusy{nullptr};
    std::uint64_t* d_ptot{nullptr};
    std::uint64_t* d_ctot{nullptr};
    std::uint64_t* d_seq{nullptr};
    DevReport* d_rep{nullptr};  // two: the report, then the disorder word
    DevReport* h_rep{nullptr};  // pinned, the same two
    std::uint64_t* d_rep_parts{nullptr};  // report partials
    std::uint32_t* d_disorder{nullptr};  // a run's records went back in time
    // scratch
    std::size_t tile_cap{0};
    PlaneSum* d_psum{nullptr};
    MaskWord* d_tmask{nullptr};  // touched planes per tile
    ChanSum* d_csum{nullptr};
    PlaneCarry* d_pcarry{nullptr};
    std::uint64_t* d_ccarry{nullptr};
    std::uint64_t* d_tcount{nullptr};
    std::uint64_t* d_tseq{nullptr};
    PlaneSum* d_gpsum{nullptr};
    ChanSum* d_gcsum{nullptr};
    PlaneCarry* d_gpcarry{nullptr};
    std::uint64_t* d_gccarry{nullptr};
    std::uint64_t* d_gcount{nullptr};
    std::uint64_t* d_gseq{nullptr};
    DevReport* d_tile_rep{nullptr};
    std::uint8_t* d_tsplit{nullptr};  // per tile: holds a split step
    StepDesc* d_desc{nullptr};  // per-step descriptors (records / 64)
    std::uint32_t* d_desc_rid{nullptr};  // and their range ids (hybrid runs)
    SplitDesc* d_desc_split{nullptr};    // and split steps' second runs
    std::size_t desc_cap{0};
    hipEvent_t ev[4]{};
    float last_ms[3]{0, 0, 0};
    std::uint64_t burst{0};
    // the last completed run's modeled records and page-register hits: a
    // large stream with few hits is mostly general steps, and its next run
    // takes the four-wave apply pass (results are the same either way)
    std::uint64_t last_modeled{0};
    std::uint64_t last_hits{0};
    int last_apply_waves{0};  // waves per SIMD the last run's apply pass was built for
};

// Where one run of the main pipeline keeps its per-tile and per-group
// summaries, carries, tile reports and step descriptors.
struct RunScratch {
    PlaneSum* psum;
    MaskWord* tmask;
    ChanSum* csum;
    PlaneCarry* pcarry;
    std::uint64_t* ccarry;
    std::uint64_t* tcount;
    std::uint64_t* tseq;
    PlaneSum* gpsum;
    ChanSum* gcsum;
    PlaneCarry* gpcarry;
    std::uint64_t* gccarry;
    std::uint64_t* gcount;
    std::uint64_t* gseq;
    DevReport* tile_rep;
    StepDesc* desc;
    std::uint8_t* tsplit;
};

namespace {

// Lays a run's scratch out in one buffer from `base`, each piece 256-byte
// aligned: per tile the plane summaries and carries (64 B per plane), the
// mask words (16 B per 64 planes), the channel summaries and carries (24 B
// per channel), two counters, a tile report (128 B) and a split flag (1 B);
// per group of kGroup
// tiles the same summaries and carries; and 16 B of step descriptor per 64
// records.  Returns the bytes needed; with base == nullptr it only counts.
std::size_t carve_scratch(const KArgs& a, std::size_t ntiles, std::size_t nsteps,
                          unsigned char* base, RunScratch* s)
{
    std::size_t off = 0;
    auto take = [&](auto*& ptr, std::size_t count) {
        using T = std::remove_reference_t<decltype(*ptr)>;
        off = (off + 255) & ~static_cast<std::size_t>(255);
        ptr = base != nullptr ? reinterpret_cast<T*>(base + off) : nullptr;
        off += sizeof(T) * (count == 0 ? 1 : count);
    };
    RunScratch t{};
    const std::size_t rp = a.Rp, rc = a.Rc;
    const std::size_t groups = (ntiles + kGroup - 1) / kGroup;
    take(t.psum, ntiles * rp);
    take(t.tmask, ntiles * mask_words(a));
    take(t.csum, ntiles * rc);
    take(t.pcarry, ntiles * rp);
    take(t.ccarry, ntiles * rc);
    take(t.tcount, ntiles);
    take(t.tseq, ntiles);
    take(t.gpsum, groups * rp);
    take(t.gcsum, groups * rc);
    take(t.gpcarry, groups * rp);
    take(t.gccarry, groups * rc);
    take(t.gcount, groups);
    take(t.gseq, groups);
    take(t.tile_rep, ntiles);
    take(t.desc, nsteps);
    take(t.tsplit, ntiles);
    if (s != nullptr) {
        *s = t;
    }
    return off;
}

}  // namespace

namespace {

int hip_status(hipError_t e) { return e == hipSuccess ? HBFSIM_OK : HBFSIM_CUDA_ERROR; }

template <typename T>
void hfree(T*& p)
{
    if (p != nullptr) {
        (void)hipFree(p);
        p = nullptr;
    }
}

template <typename T>
hipError_t halloc(T*& p, std::size_t count)
{
    return hipMalloc(reinterpret_cast<void**>(&p), sizeof(T) * (count == 0 ? 1 : count));
}

std::uint32_t bits_for(std::uint32_t n)
{
    std::uint32_t b = 0;
    while ((1u << b) < n) {
        ++b;
    }
    return b;
}

bool is_pow2(std::uint64_t v) { return v != 0 && (v & (v - 1)) == 0; }

std::uint32_t log2u(std::uint64_t v)
{
    std::uint32_t b = 0;
    while ((1ull << b) < v) {
        ++b;
    }
    return b;
}

void free_scratch(engine* e)
{
    hfree(e->d_psum);
    hfree(e->d_tmask);
    hfree(e->d_csum);
    hfree(e->d_pcarry);
    hfree(e->d_ccarry);
    hfree(e->d_tcount);
    hfree(e->d_tseq);
    hfree(e->d_gpsum);
    hfree(e->d_gcsum);
    hfree(e->d_gpcarry);
    hfree(e->d_gccarry);
    hfree(e->d_gcount);
    hfree(e->d_gseq);
    hfree(e->d_tile_rep);
    hfree(e->d_tsplit);
    hfree(e->d_desc);
    hfree(e->d_desc_rid);
    hfree(e->d_desc_split);
    e->desc_cap = 0;
    e->tile_cap = 0;
}

int ensure_scratch(engine* e, std::size_t ntiles)
{
    if (ntiles <= e->tile_cap) {
        return HBFSIM_OK;
    }
    free_scratch(e);
    // an eighth of headroom, so that batches a little larger than the last
    // do not reallocate (freeing device memory synchronises the device)
    const std::size_t cap = std::max<std::size_t>(ntiles + ntiles / 8, 16);
    const std::size_t rp = e->args.Rp, rc = e->args.Rc;
    if (halloc(e->d_psum, cap * rp) != hipSuccess ||
        halloc(e->d_tmask, cap * mask_words(e->args)) != hipSuccess ||
        halloc(e->d_csum, cap * rc) != hipSuccess ||
        halloc(e->d_pcarry, cap * rp) != hipSuccess ||
        halloc(e->d_ccarry, cap * rc) != hipSuccess || halloc(e->d_tcount, cap) != hipSuccess ||
        halloc(e->d_tseq, cap) != hipSuccess) {
        free_scratch(e);
        return HBFSIM_CUDA_ERROR;
    }
    const std::size_t gcap = (cap + kGroup - 1) / kGroup;
    if (halloc(e->d_gpsum, gcap * rp) != hipSuccess || halloc(e->d_gcsum, gcap * rc) != hipSuccess ||
        halloc(e->d_gpcarry, gcap * rp) != hipSuccess ||
        halloc(e->d_gccarry, gcap * rc) != hipSuccess || halloc(e->d_gcount, gcap) != hipSuccess ||
        halloc(e->d_gseq, gcap) != hipSuccess || halloc(e->d_tile_rep, cap) != hipSuccess ||
        halloc(e->d_tsplit, cap) != hipSuccess) {
        free_scratch(e);
        return HBFSIM_CUDA_ERROR;
    }
    e->tile_cap = cap;
    return HBFSIM_OK;
}

int upload_ranges(engine* e, hipStream_t stream)
{
    const std::size_t count = e->ranges.size();
    if (count > e->range_cap || e->d_r_base == nullptr) {
        hfree(e->d_r_base);
        hfree(e->d_r_length);
        hfree(e->d_r_offset);
        hfree(e->d_r_meta);
        hfree(e->d_r_id);
        const std::size_t cap = std::max<std::size_t>(count, 64);
        if (halloc(e->d_r_base, cap) != hipSuccess || halloc(e->d_r_length, cap) != hipSuccess ||
            halloc(e->d_r_offset, cap) != hipSuccess || halloc(e->d_r_meta, cap) != hipSuccess ||
            halloc(e->d_r_id, cap) != hipSuccess) {
            return HBFSIM_CUDA_ERROR;
        }
        e->range_cap = cap;
    }
    std::vector<std::uint64_t> base(count), length(count), offset(count);
    std::vector<std::uint32_t> meta(count), id(count);
    for (std::size_t i = 0; i < count; ++i) {
        base[i] = e->ranges[i].base;
        length[i] = e->ranges[i].length;
        offset[i] = e->ranges[i].file_offset;
        meta[i] = (e->ranges[i].mode & 0xffu) | (e->ranges[i].permissions << 8);
        id[i] = e->ranges[i].range_id;
    }
    if (count != 0) {
        hipError_t err = hipMemcpyAsync(e->d_r_base, base.data(), count * 8,
                                        hipMemcpyHostToDevice, stream);
        if (err == hipSuccess)
            err = hipMemcpyAsync(e->d_r_length, length.data(), count * 8, hipMemcpyHostToDevice,
                                 stream);
        if (err == hipSuccess)
            err = hipMemcpyAsync(e->d_r_offset, offset.data(), count * 8, hipMemcpyHostToDevice,
                                 stream);
        if (err == hipSuccess)
            err = hipMemcpyAsync(e->d_r_meta, meta.data(), count * 4, hipMemcpyHostToDevice,
                                 stream);
        if (err == hipSuccess)
            err = hipMemcpyAsync(e->d_r_id, id.data(), count * 4, hipMemcpyHostToDevice, stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
        if (err != hipSuccess) {
            return HBFSIM_CUDA_ERROR;
        }
    }
    KArgs& a = e->args;
    a.r_base = e->d_r_base;
    a.r_length = e->d_r_length;
    a.r_file_offset = e->d_r_offset;
    a.r_meta = e->d_r_meta;
    a.r_id = e->d_r_id;
    a.r_count = static_cast<std::uint32_t>(count);
    a.r_stride = count <= kMaxFences ? 1u
                                     : static_cast<std::uint32_t>((count + kMaxFences - 1) /
                                                                  kMaxFences);
    a.r_nfence = count == 0 ? 0u
                            : static_cast<std::uint32_t>((count + a.r_stride - 1) / a.r_stride);
    e->ranges_dirty = false;
    return HBFSIM_OK;
}

// Modeled records per (window of issue time, die), for the thermal power
// map.  Each block histograms a chunk in LDS over the windows it spans and
// flushes the non-zero bins with global atomics.
constexpr std::uint32_t kCountChunk = 4096;
constexpr std::uint32_t kCountBins = 4096;

__global__ __launch_bounds__(256) void k_window_counts(KArgs a, const hbf_record32* rec,
                                                       std::size_t n, std::uint64_t window_ps,
                                                       std::uint64_t windows,
                                                       std::uint32_t ndie,
                                                       std::uint32_t* counts)
{
    extern __shared__ std::uint64_t sm[];
    std::uint64_t* fence = sm;
    std::uint32_t* hist = reinterpret_cast<std::uint32_t*>(fence + a.r_nfence);
    const int tid = threadIdx.x;
    for (std::uint32_t j = tid; j < a.r_nfence; j += blockDim.x) {
        fence[j] = a.r_base[static_cast<std::size_t>(j) * a.r_stride];
    }
    for (std::uint32_t j = tid; j < kCountBins; j += blockDim.x) {
        hist[j] = 0;
    }
    __syncthreads();
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kCountChunk;
    const std::size_t end = begin + kCountChunk < n ? begin + kCountChunk : n;
    const std::uint64_t w0 = rec[begin].issue_ps / window_ps;
    RangeCache rc = empty_cache();
    for (std::size_t i = begin + tid; i < end; i += blockDim.x) {
        uint4 x, y;
        load_record(rec, i, x, y);
        const Dec d = decode<false>(a, fence, rc, x, y, 0);
        if (d.cls != kClsModeled) {
            continue;
        }
        const std::uint64_t w = d.issue / window_ps;
        if (w >= windows) {
            continue;
        }
        const std::uint32_t die = d.plane / a.P;
        const std::uint64_t bin = (w - w0) * ndie + die;
        if (w >= w0 && bin < kCountBins) {
            atomicAdd(&hist[bin], 1u);
        } else {
            atomicAdd(&counts[w * ndie + die], 1u);
        }
    }
    __syncthreads();
    for (std::uint32_t j = tid; j < kCountBins; j += blockDim.x) {
        if (hist[j] != 0) {
            atomicAdd(&counts[w0 * ndie + j], hist[j]);
        }
    }
}

// ---- empirical single-tail model (hbf_device.cu:796-881) -----------------
// One busy-until tail; a read's service is the cumulative curve's increment
// at its burst run (streak of consecutive ascending pages with one
// operation, capped at 1023, hbf_device.cuh:1031-1080), a write's is tPROG.
// Three scans over tiles of 4096 records (256 threads x 16 consecutive
// records): the streak summaries (associative, below) give every tile its
// incoming burst state; with services known, the tail's (max,+) maps give
// every tile its incoming busy time; the apply pass replays each thread's
// records from both.  Services per run come from a 1024-entry table.
constexpr int kEmpThreads = 256;
constexpr std::uint32_t kEmpPer = 16;
constexpr std::uint32_t kEmpTile = kEmpThreads * kEmpPer;
constexpr std::uint64_t kRunCap = 1023;
constexpr std::uint64_t kMaxEmpPage = (1ull << 53) - 2;

struct alignas(16) Burst {
    std::uint64_t fpage, lpage;  // first / last page of the streak records
    std::uint64_t lead, tail;    // lengths of the first and last streaks
    std::uint64_t nburst;        // records taking part in streaks
    std::uint64_t nmod;          // modeled records
    std::uint32_t fop, lop, all, pad;
};
struct alignas(16) BState {
    std::uint64_t page, run;
    std::uint32_t op, valid;
};
struct alignas(16) TailMap {
    std::uint64_t A, B;  // b -> max(b + A, B)
};

__device__ __forceinline__ Burst burst_zero()
{
    Burst b;
    b.fpage = b.lpage = b.lead = b.tail = b.nburst = b.nmod = 0;
    b.fop = b.lop = b.all = b.pad = 0;
    return b;
}

// a then b
__device__ __forceinline__ Burst burst_combine(const Burst& a, const Burst& b)
{
    if (b.nburst == 0) {
        Burst r = a;
        r.nmod = a.nmod + b.nmod;
        return r;
    }
    if (a.nburst == 0) {
        Burst r = b;
        r.nmod = a.nmod + b.nmod;
        return r;
    }
    const bool cont = a.lop == b.fop && a.lpage + 1 == b.fpage;
    Burst r;
    r.fpage = a.fpage;
    r.fop = a.fop;
    r.lpage = b.lpage;
    r.lop = b.lop;
    r.lead = (a.all && cont) ? a.lead + b.lead : a.lead;
    r.tail = (b.all && cont) ? a.tail + b.tail : b.tail;
    r.all = (a.all && b.all && cont) ? 1u : 0u;
    r.nburst = a.nburst + b.nburst;
    r.nmod = a.nmod + b.nmod;
    r.pad = 0;
    return r;
}

__device__ __forceinline__ BState burst_apply(const BState& st, const Burst& s)
{
    if (s.nburst == 0) {
        return st;
    }
    const bool cont = st.valid && st.op == s.fop && st.page + 1 == s.fpage;
    BState r;
    r.page = s.lpage;
    r.op = s.lop;
    r.valid = 1;
    const std::uint64_t len = (s.all && cont) ? st.run + s.tail : s.tail;
    r.run = len < kRunCap ? len : kRunCap;
    return r;
}

__device__ __forceinline__ void burst_add(Burst& b, std::uint64_t page, std::uint32_t op)
{
    if (b.nburst == 0) {
        b.fpage = b.lpage = page;
        b.fop = b.lop = op;
        b.lead = b.tail = 1;
        b.all = 1;
    } else {
        const bool cont = b.lop == op && b.lpage + 1 == page;
        if (cont) {
            ++b.tail;
            if (b.all) {
                ++b.lead;
            }
        } else {
            b.all = 0;
            b.tail = 1;
        }
        b.lpage = page;
        b.lop = op;
    }
    ++b.nburst;
}

// One modeled record through the burst state (orc_update_empirical_burst):
// its service in ps.
__device__ __forceinline__ std::uint64_t emp_step(BState& st, std::uint64_t page,
                                                  std::uint32_t op, const std::uint64_t* svc_ps,
                                                  std::uint64_t program_ps)
{
    if (page > kMaxEmpPage) {
        return 0;
    }
    const bool cont = st.valid && st.op == op && st.page + 1 == page;
    const std::uint64_t run = cont ? (st.run < kRunCap ? st.run + 1 : kRunCap) : 1;
    st.page = page;
    st.op = op;
    st.run = run;
    st.valid = 1;
    return op == 0 ? svc_ps[run] : program_ps;
}

__device__ __forceinline__ TailMap tail_compose(const TailMap& f, const TailMap& s)
{
    const std::uint64_t b = f.B + s.A;
    return TailMap{f.A + s.A, b > s.B ? b : s.B};
}

// Inclusive scan over the block's threads, in thread order.
template <class T, class F>
__device__ T block_scan_incl(T v, T* buf, F op)
{
    const int t = threadIdx.x;
    buf[t] = v;
    __syncthreads();
    for (int o = 1; o < kEmpThreads; o <<= 1) {
        T x = buf[t];
        if (t >= o) {
            x = op(buf[t - o], x);
        }
        __syncthreads();
        buf[t] = x;
        __syncthreads();
    }
    return buf[t];
}

struct EmpRec {
    Dec d;
    bool valid, modeled;
};

__device__ __forceinline__ EmpRec emp_decode(const KArgs& a, const std::uint64_t* fence,
                                             RangeCache& rc, const hbf_record32* rec,
                                             std::size_t n, std::size_t i, std::uint64_t base_ps)
{
    EmpRec r;
    r.valid = i < n;
    if (r.valid) {
        uint4 x, y;
        load_record(rec, i, x, y);
        r.d = decode<false>(a, fence, rc, x, y, base_ps);
    } else {
        r.d = invalid_dec();
    }
    r.modeled = r.valid && r.d.cls == kClsModeled;
    return r;
}

__device__ __forceinline__ void emp_load_fences(const KArgs& a, std::uint64_t* fence)
{
    for (std::uint32_t j = threadIdx.x; j < a.r_nfence; j += kEmpThreads) {
        fence[j] = a.r_base[static_cast<std::size_t>(j) * a.r_stride];
    }
}

// The burst summary of this thread's records, and the block's.
__device__ Burst emp_thread_burst(const KArgs& a, const std::uint64_t* fence,
                                  const hbf_record32* rec, std::size_t n, std::size_t begin,
                                  std::uint64_t base_ps)
{
    RangeCache rc = empty_cache();
    Burst b = burst_zero();
    for (std::uint32_t k = 0; k < kEmpPer; ++k) {
        const EmpRec r = emp_decode(a, fence, rc, rec, n, begin + k, base_ps);
        if (r.modeled) {
            ++b.nmod;
            const std::uint64_t page = r.d.page1 - 1;
            if (page <= kMaxEmpPage) {
                burst_add(b, page, dec_op(r.d.bits));
            }
        }
    }
    return b;
}

__global__ __launch_bounds__(kEmpThreads) void k_emp_burst(KArgs a, const hbf_record32* rec,
                                                           std::size_t n, std::uint64_t base_ps,
                                                           Burst* tiles)
{
    extern __shared__ std::uint64_t fence[];
    __shared__ Burst buf[kEmpThreads];
    emp_load_fences(a, fence);
    __syncthreads();
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kEmpTile + threadIdx.x * kEmpPer;
    const Burst b = emp_thread_burst(a, fence, rec, n, begin, base_ps);
    const Burst incl = block_scan_incl(b, buf, burst_combine);
    if (threadIdx.x == kEmpThreads - 1) {
        tiles[blockIdx.x] = incl;
    }
}

// One block: the burst state and modeled-request sequence before every
// tile, and after the last.
__global__ __launch_bounds__(kEmpThreads) void k_emp_burst_carry(const Burst* tiles,
                                                                 std::size_t ntiles, BState init,
                                                                 std::uint64_t seq0,
                                                                 BState* tile_in,
                                                                 std::uint64_t* tile_seq,
                                                                 BState* final_state,
                                                                 std::uint64_t* final_seq)
{
    __shared__ Burst buf[kEmpThreads];
    const std::size_t per = (ntiles + kEmpThreads - 1) / kEmpThreads;
    const std::size_t b = threadIdx.x * per;
    const std::size_t e = b + per < ntiles ? b + per : ntiles;
    Burst m = burst_zero();
    for (std::size_t t = b; t < e; ++t) {
        m = burst_combine(m, tiles[t]);
    }
    const Burst incl = block_scan_incl(m, buf, burst_combine);
    Burst ex = burst_zero();
    if (threadIdx.x > 0) {
        ex = buf[threadIdx.x - 1];
    }
    BState st = burst_apply(init, ex);
    std::uint64_t seq = seq0 + ex.nmod;
    for (std::size_t t = b; t < e; ++t) {
        tile_in[t] = st;
        tile_seq[t] = seq;
        st = burst_apply(st, tiles[t]);
        seq += tiles[t].nmod;
    }
    if (threadIdx.x == kEmpThreads - 1) {
        *final_state = burst_apply(init, incl);
        *final_seq = seq0 + incl.nmod;
    }
}

// Per thread: burst state at its first record (block scan of the thread
// summaries from the tile's incoming state); returns it and the number of
// modeled records before the thread within the tile.
__device__ BState emp_thread_state(const KArgs& a, const std::uint64_t* fence,
                                   const hbf_record32* rec, std::size_t n, std::size_t begin,
                                   std::uint64_t base_ps, const BState& tile_state, Burst* buf,
                                   std::uint64_t& nmod_before)
{
    const Burst mine = emp_thread_burst(a, fence, rec, n, begin, base_ps);
    block_scan_incl(mine, buf, burst_combine);
    Burst ex = burst_zero();
    if (threadIdx.x > 0) {
        ex = buf[threadIdx.x - 1];
    }
    nmod_before = ex.nmod;
    return burst_apply(tile_state, ex);
}

__device__ TailMap emp_thread_map(const KArgs& a, const std::uint64_t* fence,
                                  const hbf_record32* rec, std::size_t n, std::size_t begin,
                                  std::uint64_t base_ps, BState st, const std::uint64_t* svc_ps,
                                  std::uint64_t program_ps)
{
    RangeCache rc = empty_cache();
    TailMap m{0, 0};
    for (std::uint32_t k = 0; k < kEmpPer; ++k) {
        const EmpRec r = emp_decode(a, fence, rc, rec, n, begin + k, base_ps);
        if (r.modeled) {
            const std::uint64_t svc =
                emp_step(st, r.d.page1 - 1, dec_op(r.d.bits), svc_ps, program_ps);
            m = tail_compose(m, TailMap{svc, r.d.issue + svc});
        }
    }
    return m;
}

__global__ __launch_bounds__(kEmpThreads) void k_emp_map(KArgs a, const hbf_record32* rec,
                                                         std::size_t n, std::uint64_t base_ps,
                                                         const BState* tile_in,
                                                         const std::uint64_t* svc_ps,
                                                         std::uint64_t program_ps,
                                                         TailMap* tiles)
{
    extern __shared__ std::uint64_t fence[];
    __shared__ Burst buf[kEmpThreads];
    __shared__ TailMap mbuf[kEmpThreads];
    emp_load_fences(a, fence);
    __syncthreads();
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kEmpTile + threadIdx.x * kEmpPer;
    std::uint64_t before = 0;
    const BState st = emp_thread_state(a, fence, rec, n, begin, base_ps, tile_in[blockIdx.x], buf,
                                       before);
    const TailMap m = emp_thread_map(a, fence, rec, n, begin, base_ps, st, svc_ps, program_ps);
    const TailMap incl = block_scan_incl(m, mbuf, tail_compose);
    if (threadIdx.x == kEmpThreads - 1) {
        tiles[blockIdx.x] = incl;
    }
}

// One block: the tail before every tile and after the last.
__global__ __launch_bounds__(kEmpThreads) void k_emp_tail_carry(const TailMap* tiles,
                                                                std::size_t ntiles,
                                                                std::uint64_t tail0,
                                                                std::uint64_t* tile_tail,
                                                                std::uint64_t* final_tail)
{
    __shared__ TailMap buf[kEmpThreads];
    const std::size_t per = (ntiles + kEmpThreads - 1) / kEmpThreads;
    const std::size_t b = threadIdx.x * per;
    const std::size_t e = b + per < ntiles ? b + per : ntiles;
    TailMap m{0, 0};
    for (std::size_t t = b; t < e; ++t) {
        m = tail_compose(m, tiles[t]);
    }
    const TailMap incl = block_scan_incl(m, buf, tail_compose);
    std::uint64_t g = tail0;
    if (threadIdx.x > 0) {
        const TailMap ex = buf[threadIdx.x - 1];
        g = umax64(tail0 + ex.A, ex.B);
    }
    for (std::size_t t = b; t < e; ++t) {
        tile_tail[t] = g;
        g = umax64(g + tiles[t].A, tiles[t].B);
    }
    if (threadIdx.x == kEmpThreads - 1) {
        *final_tail = umax64(tail0 + incl.A, incl.B);
    }
}

__global__ __launch_bounds__(kEmpThreads) void k_emp_apply(
    KArgs a, const hbf_record32* rec, std::size_t n, std::uint64_t base_ps, const BState* tile_in,
    const std::uint64_t* tile_seq, const std::uint64_t* tile_tail, const std::uint64_t* svc_ps,
    std::uint64_t program_ps, std::uint64_t* completion, std::uint8_t* status, DevReport* tile_rep)
{
    extern __shared__ std::uint64_t fence[];
    __shared__ Burst buf[kEmpThreads];
    __shared__ TailMap mbuf[kEmpThreads];
    emp_load_fences(a, fence);
    __syncthreads();
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kEmpTile + threadIdx.x * kEmpPer;
    std::uint64_t before = 0;
    BState st = emp_thread_state(a, fence, rec, n, begin, base_ps, tile_in[blockIdx.x], buf,
                                 before);
    const TailMap mine = emp_thread_map(a, fence, rec, n, begin, base_ps, st, svc_ps, program_ps);
    block_scan_incl(mine, mbuf, tail_compose);
    std::uint64_t tail = tile_tail[blockIdx.x];
    if (threadIdx.x > 0) {
        const TailMap ex = mbuf[threadIdx.x - 1];
        tail = umax64(tail + ex.A, ex.B);
    }
    std::uint64_t seq = tile_seq[blockIdx.x] + before;
    unsigned long long v[14] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    RangeCache rc = empty_cache();
    for (std::uint32_t k = 0; k < kEmpPer; ++k) {
        const std::size_t i = begin + k;
        const EmpRec r = emp_decode(a, fence, rc, rec, n, i, base_ps);
        if (!r.valid) {
            break;
        }
        ++v[R_RECORDS];
        std::uint8_t sb = static_cast<std::uint8_t>(r.d.cls);
        std::uint64_t done;
        if (r.d.cls == kClsBypass) {
            done = r.d.issue;
            ++v[R_BYPASS];
        } else if (r.d.cls == kClsUnsupported) {
            done = ~0ull;
            ++v[R_UNSUPPORTED];
        } else {
            const std::uint32_t op = dec_op(r.d.bits);
            const std::uint64_t page = r.d.page1 - 1;
            if (a.hybrid) {
                const std::uint64_t key = (page << a.page_shift) ^
                                          (static_cast<std::uint64_t>(r.d.range_id) << 32) ^ op;
                if (seq < a.hybrid_warmup ||
                    (a.hybrid_threshold != 0 && mix64(seq ^ key) <= a.hybrid_threshold)) {
                    sb |= 8u;
                    ++v[R_HYBRID];
                }
            }
            ++seq;
            const std::uint64_t svc = emp_step(st, page, op, svc_ps, program_ps);
            done = umax64(tail, r.d.issue) + svc;
            tail = done;
            ++v[R_MODELED];
            ++v[op == 0 ? R_READS : R_WRITES];
            v[R_MAKESPAN] = umax64(v[R_MAKESPAN], done);
            const std::uint64_t lat = done - r.d.issue;
            const unsigned long long lo = v[R_LAT_LO] + lat;
            v[R_LAT_HI] += lo < v[R_LAT_LO] ? 1u : 0u;
            v[R_LAT_LO] = lo;
            v[R_LAT_MAX] = umax64(v[R_LAT_MAX], lat);
            v[R_SERVICE] += svc;
        }
        put_done(&completion[i], done);
        if (status != nullptr) {
            status[i] = sb;
        }
    }
    // block report
    __shared__ unsigned long long part[kEmpThreads * 14];
    for (int k = 0; k < 14; ++k) {
        part[threadIdx.x * 14 + k] = v[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        DevReport out{};
        for (int t = 0; t < kEmpThreads; ++t) {
            const unsigned long long* q = part + t * 14;
            for (int k = 0; k < 14; ++k) {
                if (k == R_MAKESPAN || k == R_LAT_MAX) {
                    out.v[k] = umax64(out.v[k], q[k]);
                } else if (k == R_LAT_LO) {
                    const unsigned long long s2 = out.v[k] + q[k];
                    out.v[R_LAT_HI] += s2 < out.v[k] ? 1u : 0u;
                    out.v[k] = s2;
                } else {
                    out.v[k] += q[k];
                }
            }
        }
        tile_rep[blockIdx.x] = out;
    }
}

// ---- two page registers per plane (device_coalescer.cpp:134-168) ---------
// A miss fills the first empty slot, else slot 0.  Slot 1 is therefore
// written once and then kept, and from then on a read hits when its page is
// slot 1's or the last page other than slot 1's seen on the plane.  Hits do
// not depend on timing, so they come from their own scans and the timing
// pipeline consumes them (kHits):
//   k_k2_first   per plane, the first record (optionally: whose page differs
//                from a given one) -- the fill events before both slots hold
//                a page; only run while some plane has an empty slot;
//   k_k2_last    per tile and plane, the last page other than slot 1's;
//   k_k2_up/mid/down  the carry of that page across tiles;
//   k_k2_hits    one hit byte per record.
struct K2Plane {
    std::uint64_t start3;  // first record index with both slots held
    std::uint64_t miss1, miss2;  // fill events before that (or ~0)
    std::uint32_t t1;      // slot 1's page + 1 from start3 on (0: never)
    std::uint32_t l_init;  // last page other than t1 before the run
};

constexpr std::uint32_t kK2Chunk = 16384;

__global__ __launch_bounds__(256) void k_k2_first(KArgs a, const hbf_record32* rec,
                                                  std::size_t n, std::uint64_t base_ps,
                                                  const std::uint32_t* want,
                                                  const std::uint32_t* differ,
                                                  unsigned long long* first)
{
    extern __shared__ std::uint64_t sm[];
    std::uint64_t* fence = sm;
    unsigned long long* lmin = reinterpret_cast<unsigned long long*>(fence + a.r_nfence);
    for (std::uint32_t j = threadIdx.x; j < a.r_nfence; j += blockDim.x) {
        fence[j] = a.r_base[static_cast<std::size_t>(j) * a.r_stride];
    }
    for (std::uint32_t r = threadIdx.x; r < a.Rp; r += blockDim.x) {
        lmin[r] = ~0ull;
    }
    __syncthreads();
    const std::size_t begin = static_cast<std::size_t>(blockIdx.x) * kK2Chunk;
    const std::size_t end = begin + kK2Chunk < n ? begin + kK2Chunk : n;
    RangeCache rc = empty_cache();
    for (std::size_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        uint4 x, y;
        load_record(rec, i, x, y);
        const Dec d = decode<false>(a, fence, rc, x, y, base_ps);
        if (d.cls != kClsModeled || !want[d.plane]) {
            continue;
        }
        const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
        if (differ[d.plane] != 0 && page1 == differ[d.plane]) {
            continue;
        }
        atomicMin(&lmin[d.plane], static_cast<unsigned long long>(i));
    }
    __syncthreads();
    for (std::uint32_t r = threadIdx.x; r < a.Rp; r += blockDim.x) {
        if (lmin[r] != ~0ull) {
            atomicMin(&first[r], lmin[r]);
        }
    }
}

// Page + 1 of record idx[r] for every plane r (0 when none).
__global__ __launch_bounds__(256) void k_k2_page(KArgs a, const hbf_record32* rec, std::size_t n,
                                                 std::uint64_t base_ps,
                                                 const unsigned long long* idx,
                                                 std::uint32_t* page1)
{
    extern __shared__ std::uint64_t fence[];
    for (std::uint32_t j = threadIdx.x; j < a.r_nfence; j += blockDim.x) {
        fence[j] = a.r_base[static_cast<std::size_t>(j) * a.r_stride];
    }
    __syncthreads();
    for (std::uint32_t r = threadIdx.x; r < a.Rp; r += blockDim.x) {
        std::uint32_t v = 0;
        if (idx[r] < n) {
            RangeCache rc = empty_cache();
            uint4 x, y;
            load_record(rec, idx[r], x, y);
            v = static_cast<std::uint32_t>(decode<false>(a, fence, rc, x, y, base_ps).page1);
        }
        page1[r] = v;
    }
}

__global__ __launch_bounds__(64) void k_k2_last(KArgs a, const hbf_record32* rec, std::size_t n,
                                                std::uint64_t base_ps, const K2Plane* kp,
                                                std::uint32_t* tile_last)
{
    extern __shared__ std::uint64_t sm[];
    std::uint64_t* fence = sm;
    std::uint32_t* t1 = reinterpret_cast<std::uint32_t*>(fence + a.r_nfence);
    std::uint32_t* last = t1 + a.Rp;
    const int lane = threadIdx.x;
    load_fences(a, fence, lane);
    for (std::uint32_t r = lane; r < a.Rp; r += kWave) {
        t1[r] = kp[r].t1;
        last[r] = 0;
    }
    __syncthreads();
    const std::size_t tile = blockIdx.x;
    const std::size_t begin = tile * a.tile;
    const std::size_t end = begin + a.tile < n ? begin + a.tile : n;
    RangeCache rc = empty_cache();
    for (std::size_t s = begin; s < end; s += kWave) {
        const std::size_t i = s + lane;
        const bool valid = i < end;
        Dec d = invalid_dec();
        if (valid) {
            uint4 x, y;
            load_record(rec, i, x, y);
            d = decode<false>(a, fence, rc, x, y, base_ps);
        }
        const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
        const bool nt = valid && d.cls == kClsModeled && page1 != t1[d.plane];
        const std::uint64_t active = __ballot(nt);
        if (active == 0) {
            continue;
        }
        const Group g = group_by(nt ? d.plane : 0u, a.pbits, nt, active, lane);
        if (nt && lane == g.last) {
            last[d.plane] = page1;
        }
    }
    __syncthreads();
    for (std::uint32_t r = lane; r < a.Rp; r += kWave) {
        tile_last[tile * a.Rp + r] = last[r];
    }
}

// Level 1: the last nonzero page of each (group of kGroup tiles, plane).
__global__ __launch_bounds__(256) void k_k2_up(KArgs a, std::size_t ntiles, std::size_t ngroups,
                                               const std::uint32_t* tile_last,
                                               std::uint32_t* group_last)
{
    const std::size_t t = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
    if (t >= ngroups * a.Rp) {
        return;
    }
    const std::size_t g = t / a.Rp, r = t % a.Rp;
    std::uint32_t v = 0;
    const std::size_t e = (g + 1) * kGroup < ntiles ? (g + 1) * kGroup : ntiles;
    for (std::size_t k = g * kGroup; k < e; ++k) {
        const std::uint32_t x = tile_last[k * a.Rp + r];
        v = x != 0 ? x : v;
    }
    group_last[g * a.Rp + r] = v;
}

// Level 2: per plane, the page before each group, and after the last.
__global__ __launch_bounds__(256) void k_k2_mid(KArgs a, std::size_t ngroups, const K2Plane* kp,
                                                const std::uint32_t* group_last,
                                                std::uint32_t* group_in, std::uint32_t* final_last)
{
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.Rp) {
        return;
    }
    std::uint32_t v = kp[r].l_init;
    for (std::size_t g = 0; g < ngroups; ++g) {
        group_in[g * a.Rp + r] = v;
        const std::uint32_t x = group_last[g * a.Rp + r];
        v = x != 0 ? x : v;
    }
    final_last[r] = v;
}

// Level 3: the page before each tile.
__global__ __launch_bounds__(256) void k_k2_down(KArgs a, std::size_t ntiles, std::size_t ngroups,
                                                 const std::uint32_t* tile_last,
                                                 const std::uint32_t* group_in,
                                                 std::uint32_t* tile_in)
{
    const std::size_t t = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
    if (t >= ngroups * a.Rp) {
        return;
    }
    const std::size_t g = t / a.Rp, r = t % a.Rp;
    std::uint32_t v = group_in[g * a.Rp + r];
    const std::size_t e = (g + 1) * kGroup < ntiles ? (g + 1) * kGroup : ntiles;
    for (std::size_t k = g * kGroup; k < e; ++k) {
        tile_in[k * a.Rp + r] = v;
        const std::uint32_t x = tile_last[k * a.Rp + r];
        v = x != 0 ? x : v;
    }
}

__global__ __launch_bounds__(64) void k_k2_hits(KArgs a, const hbf_record32* rec, std::size_t n,
                                                std::uint64_t base_ps, const K2Plane* kp,
                                                const std::uint32_t* tile_in, std::uint8_t* hits)
{
    extern __shared__ std::uint64_t sm[];
    std::uint64_t* fence = sm;
    std::uint32_t* t1 = reinterpret_cast<std::uint32_t*>(fence + a.r_nfence);
    std::uint32_t* last = t1 + a.Rp;
    const int lane = threadIdx.x;
    const std::size_t tile = blockIdx.x;
    load_fences(a, fence, lane);
    for (std::uint32_t r = lane; r < a.Rp; r += kWave) {
        t1[r] = kp[r].t1;
        last[r] = tile_in[tile * a.Rp + r];
    }
    __syncthreads();
    const std::size_t begin = tile * a.tile;
    const std::size_t end = begin + a.tile < n ? begin + a.tile : n;
    RangeCache rc = empty_cache();
    for (std::size_t s = begin; s < end; s += kWave) {
        const std::size_t i = s + lane;
        const bool valid = i < end;
        Dec d = invalid_dec();
        if (valid) {
            uint4 x, y;
            load_record(rec, i, x, y);
            d = decode<false>(a, fence, rc, x, y, base_ps);
        }
        const bool m = valid && d.cls == kClsModeled;
        const std::uint32_t page1 = static_cast<std::uint32_t>(d.page1);
        const std::uint32_t pt1 = m ? t1[d.plane] : 0u;
        const bool nt = m && page1 != pt1;
        const std::uint64_t active = __ballot(nt);
        bool hit = false;
        if (active != 0) {
            const Group g = group_by(nt ? d.plane : 0u, a.pbits, nt, active, lane);
            std::uint32_t prev1 = static_cast<std::uint32_t>(
                __shfl(static_cast<int>(page1), g.pred < 0 ? lane : g.pred));
            if (g.pred < 0) {
                prev1 = nt ? last[d.plane] : 0u;
            }
            hit = nt && prev1 == page1;
            __syncthreads();  // every lane has read `last` before it changes
            if (nt && lane == g.last) {
                last[d.plane] = page1;
            }
            __syncthreads();
        }
        if (m) {
            const K2Plane& k = kp[d.plane];
            if (i < k.start3) {
                hit = i != k.miss1 && i != k.miss2;
            } else if (!nt) {
                hit = true;  // slot 1's page
            }
            hits[i] = hit ? 1u : 0u;
        } else if (valid) {
            hits[i] = 0;
        }
    }
}

std::size_t lds_summary(const KArgs& a)
{
    return summary_stripe_offset(a) + (a.stripe_lds ? 4ull * a.Rp : 0ull);
}

std::size_t lds_apply(const KArgs& a)
{
    return apply_stripe_offset(a) + (a.stripe_lds ? 4ull * a.Rp : 0ull);
}

// The lane-matching tables go where they cost neither per-record pass any
// waves per CU (gfx950: 160 KB of LDS per CU, four SIMDs; both passes run at
// most four waves per SIMD).
constexpr std::size_t kLdsPerCuBytes = 160 * 1024;  // gfx950
constexpr std::size_t kSimdsPerCu = 4;
// the four-wave apply pass is considered from this many records
constexpr std::size_t kWideApplyRecords = std::size_t{1} << 24;
// A workgroup may hold all of it; beyond 64 KB of dynamic LDS a kernel has
// to be allowed the size first (allow_lds).
constexpr std::size_t kLdsPerBlockBytes = 160 * 1024;

// Raises a kernel's dynamic-LDS limit where a launch needs more than the
// default 64 KB (geometries of more than about 1,900 planes).
template <typename F>
hipError_t allow_lds(F* kernel, std::size_t bytes)
{
    if (bytes <= 65536) {
        return hipSuccess;
    }
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

void choose_match(KArgs& a)
{
    constexpr std::size_t kLdsPerCu = kLdsPerCuBytes;
    constexpr std::size_t kMaxWaves = 4 * kSimdsPerCu;
    const auto waves = [&](std::size_t bytes) {
        const std::size_t w = bytes == 0 ? kMaxWaves : kLdsPerCu / bytes;
        return w < kMaxWaves ? w : kMaxWaves;
    };
    a.match_lds = 0;
    a.stripe_lds = 0;
    const std::size_t s0 = lds_summary(a), p0 = lds_apply(a);
    a.match_lds = 1;
    if (waves(lds_summary(a)) < waves(s0) || waves(lds_apply(a)) < waves(p0)) {
        a.match_lds = 0;
    }
    // the stripe table likewise, for power-of-two axes (plane ids below
    // 2^20 and channel ids below 2^12 pack into one word)
    if (!a.flat && a.pow2 && a.Rp <= (1u << 20) && a.Rc <= (1u << 12)) {
        const std::size_t s1 = lds_summary(a), p1 = lds_apply(a);
        a.stripe_lds = 1;
        if (waves(lds_summary(a)) < waves(s1) || waves(lds_apply(a)) < waves(p1)) {
            a.stripe_lds = 0;
        }
    }
}

// Records per tile when the configuration leaves it open: the largest power
// of two up to 16384 that gives every CU sixteen tiles, down to 1024 records;
// below that, the largest that gives every CU eight tiles, at least 256.
// (Mid-sized runs of 2^22 to 2^25 records take twice the tiles they would at
// eight per CU: more waves to cover the per-record passes' latency, at the
// price of a carry chain of twice the tiles.)
std::uint32_t auto_tile(std::size_t n)
{
    std::uint32_t t = 16384;
    while (t > 1024 && (n + t - 1) / t < 4096) {
        t >>= 1;
    }
    while (t > 256 && (n + t - 1) / t < 2048) {
        t >>= 1;
    }
    return t;
}

// Empirical curve on the host (hbf_device.cuh:959-1029), for the per-run
// service table.
std::uint64_t sat_mul(std::uint64_t a, std::uint32_t b)
{
    return b != 0 && a > ~0ull / b ? ~0ull : a * b;
}

std::uint64_t sat_add_host(std::uint64_t a, std::uint64_t b)
{
    return b > ~0ull - a ? ~0ull : a + b;
}

std::uint64_t ceiling_scaled_delta(std::uint64_t delta, std::uint32_t offset, std::uint32_t span)
{
    if (delta == 0 || offset == 0) {
        return 0;
    }
    if (span == 0) {
        return ~0ull;
    }
    const std::uint64_t q = delta / span, r = delta % span;
    return sat_add_host(sat_mul(q, offset), (r * offset + span - 1) / span);
}

std::uint64_t emp_cumulative(const engine_config& c, std::uint32_t run)
{
    if (run == 0) {
        return 0;
    }
    const std::uint32_t count = 6;
    std::uint32_t right = 0;
    while (right < count && run > c.emp_pages[right]) {
        ++right;
    }
    if (right == count) {
        right = count - 1;
    }
    std::uint32_t left_pages = 0;
    std::uint64_t left_ns = 0;
    if (right != 0) {
        left_pages = c.emp_pages[right - 1];
        left_ns = c.emp_cum_ns[right - 1];
    }
    if (run > c.emp_pages[right]) {
        left_pages = c.emp_pages[count - 2];
        left_ns = c.emp_cum_ns[count - 2];
        right = count - 1;
    }
    if (c.emp_pages[right] <= left_pages || c.emp_cum_ns[right] < left_ns || run < left_pages) {
        return ~0ull;
    }
    return sat_add_host(left_ns, ceiling_scaled_delta(c.emp_cum_ns[right] - left_ns,
                                                      run - left_pages,
                                                      c.emp_pages[right] - left_pages));
}

bool emp_control_valid(const engine_config& c)
{
    if (c.emp_program_ns == 0) {
        return false;
    }
    for (int i = 0; i < 6; ++i) {
        if (c.emp_pages[i] == 0 || c.emp_cum_ns[i] == 0 ||
            (i != 0 && (c.emp_pages[i] <= c.emp_pages[i - 1] ||
                        c.emp_cum_ns[i] <= c.emp_cum_ns[i - 1]))) {
            return false;
        }
    }
    return c.emp_pages[5] <= kRunCap;
}

// Service (ps) of a read at burst run 0..1023; products wrap like the CPU
// restatement's.
std::vector<std::uint64_t> emp_service_table(const engine_config& c)
{
    std::vector<std::uint64_t> t(kRunCap + 1, 0);
    for (std::uint32_t run = 1; run <= kRunCap; ++run) {
        const std::uint64_t cur = emp_cumulative(c, run), prev = emp_cumulative(c, run - 1);
        const std::uint64_t ns = cur < prev ? ~0ull : cur - prev;
        t[run] = ns * 1000ull;
    }
    return t;
}

int run_empirical(engine* e, const hbf_record32* d_rec, std::size_t n, std::uint64_t* d_comp,
                  std::uint8_t* d_status, std::uint64_t base_ps, hipStream_t stream,
                  hbfsim_amd_report* out, bool in_order)
{
    const engine_config& c = e->cfg;
    if (c.page_shift != 12 || !emp_control_valid(c)) {
        return HBFSIM_UNSUPPORTED;
    }
    const KArgs& a = e->args;
    const std::size_t ntiles = (n + kEmpTile - 1) / kEmpTile;
    const std::vector<std::uint64_t> table = emp_service_table(c);
    std::uint64_t* d_svc = nullptr;
    Burst* d_bt = nullptr;
    BState* d_in = nullptr;
    std::uint64_t* d_tseq = nullptr;
    TailMap* d_maps = nullptr;
    std::uint64_t* d_tail = nullptr;
    DevReport* d_trep = nullptr;
    BState* d_final = nullptr;
    std::uint64_t* d_fin = nullptr;  // [0] sequence, [1] tail
    auto release = [&]() {
        hfree(d_svc); hfree(d_bt); hfree(d_in); hfree(d_tseq); hfree(d_maps); hfree(d_tail);
        hfree(d_trep); hfree(d_final); hfree(d_fin);
    };
    hipError_t err = halloc(d_svc, table.size());
    if (err == hipSuccess) err = halloc(d_bt, ntiles);
    if (err == hipSuccess) err = halloc(d_in, ntiles);
    if (err == hipSuccess) err = halloc(d_tseq, ntiles);
    if (err == hipSuccess) err = halloc(d_maps, ntiles);
    if (err == hipSuccess) err = halloc(d_tail, ntiles);
    if (err == hipSuccess) err = halloc(d_trep, ntiles);
    if (err == hipSuccess) err = halloc(d_final, 1);
    if (err == hipSuccess) err = halloc(d_fin, 2);
    std::uint64_t seq0 = 0, tail0 = 0;
    std::uint32_t back = 0;
    const std::uint32_t zero = 0;
    if (err == hipSuccess && !in_order &&
        order_check(d_rec, false, n, e->d_disorder, stream) != HBFSIM_OK) {
        err = hipErrorLaunchFailure;
    }
    if (err == hipSuccess)
        err = hipMemcpyAsync(d_svc, table.data(), table.size() * 8, hipMemcpyHostToDevice, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(&seq0, e->d_seq, 8, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(&tail0, e->d_cbusy, 8, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(&back, e->d_disorder, 4, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err == hipSuccess && back != 0) {
        err = hipMemcpyAsync(e->d_disorder, &zero, 4, hipMemcpyHostToDevice, stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
    }
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    if (back != 0) {
        // a record's issue time goes back: served in (issue, position) order
        release();
        return run_in_issue_order(
            d_rec, false, n, d_comp, d_status, stream,
            [&](const void* sorted, std::uint64_t* comp, std::uint8_t* status) {
                return run_empirical(e, static_cast<const hbf_record32*>(sorted), n, comp, status,
                                     base_ps, stream, out, true);
            });
    }
    BState init{};
    {
        const std::uint64_t packed = e->burst;
        const std::uint64_t p1 = packed >> 11;
        init.valid = (packed != 0 && (packed & kRunCap) != 0 && p1 != 0) ? 1u : 0u;
        init.page = p1 == 0 ? 0 : p1 - 1;
        init.op = static_cast<std::uint32_t>((packed >> 10) & 1u);
        init.run = packed & kRunCap;
    }
    const std::size_t lds = 8ull * a.r_nfence;
    const dim3 grid(static_cast<unsigned>(ntiles));
    (void)hipEventRecord(e->ev[0], stream);
    hipLaunchKernelGGL(k_emp_burst, grid, dim3(kEmpThreads), lds, stream, a, d_rec, n, base_ps,
                       d_bt);
    hipLaunchKernelGGL(k_emp_burst_carry, dim3(1), dim3(kEmpThreads), 0, stream,
                       static_cast<const Burst*>(d_bt), ntiles, init, seq0, d_in, d_tseq, d_final,
                       d_fin);
    (void)hipEventRecord(e->ev[1], stream);
    hipLaunchKernelGGL(k_emp_map, grid, dim3(kEmpThreads), lds, stream, a, d_rec, n, base_ps,
                       static_cast<const BState*>(d_in), static_cast<const std::uint64_t*>(d_svc),
                       c.emp_program_ns * 1000ull, d_maps);
    hipLaunchKernelGGL(k_emp_tail_carry, dim3(1), dim3(kEmpThreads), 0, stream,
                       static_cast<const TailMap*>(d_maps), ntiles, tail0, d_tail, d_fin + 1);
    (void)hipEventRecord(e->ev[2], stream);
    hipLaunchKernelGGL(k_emp_apply, grid, dim3(kEmpThreads), lds, stream, a, d_rec, n, base_ps,
                       static_cast<const BState*>(d_in), static_cast<const std::uint64_t*>(d_tseq),
                       static_cast<const std::uint64_t*>(d_tail),
                       static_cast<const std::uint64_t*>(d_svc), c.emp_program_ns * 1000ull,
                       d_comp, d_status, d_trep);
    (void)hipEventRecord(e->ev[3], stream);
    launch_report(stream, static_cast<const DevReport*>(d_trep), ntiles, e->d_rep,
                  e->d_rep_parts, nullptr);
    BState fin{};
    std::uint64_t fin2[2] = {0, 0};
    err = hipGetLastError();
    if (err == hipSuccess)
        err = hipMemcpyAsync(e->h_rep, e->d_rep, sizeof(DevReport), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(&fin, d_final, sizeof(BState), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(fin2, d_fin, 16, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(e->d_seq, d_fin, 8, hipMemcpyDeviceToDevice, stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(e->d_cbusy, d_fin + 1, 8, hipMemcpyDeviceToDevice, stream);
    std::uint64_t tot = 0;
    if (err == hipSuccess)
        err = hipMemcpyAsync(&tot, e->d_ctot, 8, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err == hipSuccess) {
        tot += e->h_rep->v[R_SERVICE];
        err = hipMemcpyAsync(e->d_ctot, &tot, 8, hipMemcpyHostToDevice, stream);
    }
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    release();
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (fin.valid) {
        e->burst = ((fin.page + 1) << 11) | (static_cast<std::uint64_t>(fin.op) << 10) | fin.run;
    }
    for (int k = 0; k < 3; ++k) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e->ev[k], e->ev[k + 1]) == hipSuccess) {
            e->last_ms[k] = ms;
        }
    }
    if (out != nullptr) {
        std::memcpy(out, e->h_rep, sizeof(DevReport));
    }
    return HBFSIM_OK;
}

// Per-record page-buffer hits for two registers per plane, and the tags the
// run leaves behind (host array [2 * planes]).  d_hits: n bytes.
int k2_hits(engine* e, const KArgs& a, const hbf_record32* d_rec, std::size_t n,
            std::uint64_t base_ps, std::size_t ntiles, hipStream_t stream, std::uint8_t* d_hits,
            std::vector<std::uint64_t>& tags_out)
{
    const std::uint32_t rp = a.Rp;
    std::vector<std::uint64_t> tags(2ull * rp);
    hipError_t err = hipMemcpyAsync(tags.data(), e->d_ptag, tags.size() * 8,
                                    hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    std::vector<K2Plane> kp(rp);
    std::vector<std::uint32_t> want(rp, 0), differ(rp, 0);
    std::vector<unsigned long long> idx_a(rp, ~0ull), idx_b(rp, ~0ull);
    std::vector<std::uint32_t> page_a(rp, 0), page_b(rp, 0);
    bool need_a = false;
    for (std::uint32_t r = 0; r < rp; ++r) {
        const std::uint64_t t0 = tags[2 * r], t1 = tags[2 * r + 1];
        need_a = need_a || (t0 == 0 && t1 == 0);
    }
    std::uint32_t* d_want = nullptr;
    std::uint32_t* d_differ = nullptr;
    unsigned long long* d_first = nullptr;
    std::uint32_t* d_page = nullptr;
    K2Plane* d_kp = nullptr;
    const std::size_t ngroups = (ntiles + kGroup - 1) / kGroup;
    std::uint32_t* d_tlast = nullptr;
    std::uint32_t* d_tin = nullptr;
    std::uint32_t* d_glast = nullptr;
    std::uint32_t* d_gin = nullptr;
    std::uint32_t* d_final = nullptr;
    auto release = [&]() {
        hfree(d_want); hfree(d_differ); hfree(d_first); hfree(d_page); hfree(d_kp);
        hfree(d_tlast); hfree(d_tin); hfree(d_glast); hfree(d_gin); hfree(d_final);
    };
    err = halloc(d_want, rp);
    if (err == hipSuccess) err = halloc(d_differ, rp);
    if (err == hipSuccess) err = halloc(d_first, rp);
    if (err == hipSuccess) err = halloc(d_page, rp);
    if (err == hipSuccess) err = halloc(d_kp, rp);
    if (err == hipSuccess) err = halloc(d_tlast, ntiles * rp);
    if (err == hipSuccess) err = halloc(d_tin, ntiles * rp);
    if (err == hipSuccess) err = halloc(d_glast, ngroups * rp);
    if (err == hipSuccess) err = halloc(d_gin, ngroups * rp);
    if (err == hipSuccess) err = halloc(d_final, rp);
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    const unsigned first_blocks = static_cast<unsigned>((n + kK2Chunk - 1) / kK2Chunk);
    const std::size_t lds_first = 8ull * a.r_nfence + 8ull * rp;
    // pass A: the first record of every plane with both slots empty
    auto first_pass = [&](std::vector<unsigned long long>& idx,
                          std::vector<std::uint32_t>& page) -> hipError_t {
        std::vector<unsigned long long> init(rp, ~0ull);
        hipError_t e2 = hipMemcpyAsync(d_want, want.data(), rp * 4, hipMemcpyHostToDevice, stream);
        if (e2 == hipSuccess)
            e2 = hipMemcpyAsync(d_differ, differ.data(), rp * 4, hipMemcpyHostToDevice, stream);
        if (e2 == hipSuccess)
            e2 = hipMemcpyAsync(d_first, init.data(), rp * 8, hipMemcpyHostToDevice, stream);
        if (e2 != hipSuccess) return e2;
        hipLaunchKernelGGL(k_k2_first, dim3(first_blocks), dim3(256), lds_first, stream, a, d_rec,
                           n, base_ps, static_cast<const std::uint32_t*>(d_want),
                           static_cast<const std::uint32_t*>(d_differ), d_first);
        hipLaunchKernelGGL(k_k2_page, dim3(1), dim3(256), 8ull * a.r_nfence, stream, a, d_rec, n,
                           base_ps, static_cast<const unsigned long long*>(d_first), d_page);
        e2 = hipGetLastError();
        if (e2 == hipSuccess)
            e2 = hipMemcpyAsync(idx.data(), d_first, rp * 8, hipMemcpyDeviceToHost, stream);
        if (e2 == hipSuccess)
            e2 = hipMemcpyAsync(page.data(), d_page, rp * 4, hipMemcpyDeviceToHost, stream);
        if (e2 == hipSuccess) e2 = hipStreamSynchronize(stream);
        return e2;
    };
    if (need_a) {
        for (std::uint32_t r = 0; r < rp; ++r) {
            want[r] = tags[2 * r] == 0 && tags[2 * r + 1] == 0;
            differ[r] = 0;
        }
        err = first_pass(idx_a, page_a);
    }
    // pass B: the first record whose page differs from the one slot held
    if (err == hipSuccess) {
        bool any = false;
        for (std::uint32_t r = 0; r < rp; ++r) {
            const std::uint64_t t0 = tags[2 * r], t1 = tags[2 * r + 1];
            want[r] = 0;
            differ[r] = 0;
            if (t0 != 0 && t1 == 0) {
                want[r] = 1;
                differ[r] = static_cast<std::uint32_t>(t0);
            } else if (t0 == 0 && t1 != 0) {
                want[r] = 1;
                differ[r] = static_cast<std::uint32_t>(t1);
            } else if (t0 == 0 && t1 == 0 && idx_a[r] < n) {
                want[r] = 1;
                differ[r] = page_a[r];
            }
            any = any || want[r];
        }
        if (any) {
            err = first_pass(idx_b, page_b);
        }
    }
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    for (std::uint32_t r = 0; r < rp; ++r) {
        const std::uint64_t t0 = tags[2 * r], t1 = tags[2 * r + 1];
        K2Plane& k = kp[r];
        k.start3 = ~0ull;
        k.miss1 = k.miss2 = ~0ull;
        k.t1 = 0;
        k.l_init = 0;
        const bool b = idx_b[r] < n;
        if (t0 != 0 && t1 != 0) {
            k.start3 = 0;
            k.t1 = static_cast<std::uint32_t>(t1);
            k.l_init = static_cast<std::uint32_t>(t0);
        } else if (t0 != 0) {
            k.l_init = static_cast<std::uint32_t>(t0);
            if (b) {
                k.miss2 = idx_b[r];
                k.start3 = idx_b[r] + 1;
                k.t1 = page_b[r];
            }
        } else if (t1 != 0) {
            k.t1 = static_cast<std::uint32_t>(t1);
            if (b) {
                k.miss1 = idx_b[r];
                k.start3 = idx_b[r] + 1;
            }
        } else if (idx_a[r] < n) {
            k.miss1 = idx_a[r];
            if (b) {
                k.miss2 = idx_b[r];
                k.start3 = idx_b[r] + 1;
                k.t1 = page_b[r];
            }
        }
    }
    err = hipMemcpyAsync(d_kp, kp.data(), rp * sizeof(K2Plane), hipMemcpyHostToDevice, stream);
    if (err != hipSuccess) {
        release();
        return HBFSIM_CUDA_ERROR;
    }
    const std::size_t lds = 8ull * a.r_nfence + 8ull * rp;
    const unsigned wide = static_cast<unsigned>((ngroups * rp + 255) / 256);
    hipLaunchKernelGGL(k_k2_last, dim3(static_cast<unsigned>(ntiles)), dim3(kWave), lds, stream, a,
                       d_rec, n, base_ps, static_cast<const K2Plane*>(d_kp), d_tlast);
    hipLaunchKernelGGL(k_k2_up, dim3(wide), dim3(256), 0, stream, a, ntiles, ngroups,
                       static_cast<const std::uint32_t*>(d_tlast), d_glast);
    hipLaunchKernelGGL(k_k2_mid, dim3((rp + 255) / 256), dim3(256), 0, stream, a, ngroups,
                       static_cast<const K2Plane*>(d_kp), static_cast<const std::uint32_t*>(d_glast),
                       d_gin, d_final);
    hipLaunchKernelGGL(k_k2_down, dim3(wide), dim3(256), 0, stream, a, ntiles, ngroups,
                       static_cast<const std::uint32_t*>(d_tlast),
                       static_cast<const std::uint32_t*>(d_gin), d_tin);
    hipLaunchKernelGGL(k_k2_hits, dim3(static_cast<unsigned>(ntiles)), dim3(kWave), lds, stream, a,
                       d_rec, n, base_ps, static_cast<const K2Plane*>(d_kp),
                       static_cast<const std::uint32_t*>(d_tin), d_hits);
    std::vector<std::uint32_t> fin(rp);
    err = hipGetLastError();
    if (err == hipSuccess)
        err = hipMemcpyAsync(fin.data(), d_final, rp * 4, hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    release();
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    tags_out.assign(2ull * rp, 0);
    for (std::uint32_t r = 0; r < rp; ++r) {
        tags_out[2 * r] = fin[r];
        tags_out[2 * r + 1] = kp[r].t1;
    }
    return HBFSIM_OK;
}

}  // namespace

int engine_create(const engine_config& c, engine** out)
{
    *out = nullptr;
    const std::uint32_t rp = c.n_planes(), rc = c.n_channels();
    if (c.channels == 0 || c.ways == 0 || c.dies == 0 || c.planes == 0 || c.page_shift < 9 ||
        c.page_shift > 31 || c.slots > 2 || c.xfer_den == 0 || c.xfer_quantum == 0 ||
        c.tile % kWave != 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (rp > kMaxPlanes || rc > kMaxChannels) {
        return HBFSIM_UNSUPPORTED;
    }
    // bytes * num must fit 64 bits for every transfer size up to a page.
    const unsigned __int128 worst =
        static_cast<unsigned __int128>(1ull << c.page_shift) * c.xfer_num + c.xfer_den;
    if (worst > ~0ull) {
        return HBFSIM_UNSUPPORTED;
    }
    auto* e = new (std::nothrow) engine;
    if (e == nullptr) {
        return HBFSIM_IO_ERROR;
    }
    e->cfg = c;
    if (hipGetDevice(&e->device) != hipSuccess) {
        delete e;
        return HBFSIM_CUDA_ERROR;
    }
    KArgs& a = e->args;
    std::memset(&a, 0, sizeof(a));
    a.Rp = rp;
    a.Rc = rc;
    a.W = c.ways;
    a.D = c.dies;
    a.P = c.planes;
    a.pbits = bits_for(rp);
    a.cbits = bits_for(rc);
    a.flat = (rp == 1 && rc == 1) ? 1u : 0u;
    const std::uint32_t size[4] = {c.channels, c.ways, c.dies, c.planes};
    std::uint64_t div = 1;
    bool pow2 = true;
    for (int i = 0; i < 4; ++i) {
        const std::uint32_t ax = c.order[i];
        a.axis_size[ax] = size[ax];
        a.axis_div[ax] = div;
        pow2 = pow2 && is_pow2(size[ax]);
        div *= size[ax];
    }
    for (int ax = 0; ax < 4; ++ax) {
        a.axis_shift[ax] = log2u(a.axis_div[ax]);
    }
    a.pow2 = pow2 ? 1u : 0u;
    a.page_shift = c.page_shift;
    a.slots = c.slots;
    a.contention = c.contention;
    a.transfer_page = c.transfer_page;
    a.every_write = c.every_write;
    a.hybrid = c.hybrid;
    a.hybrid_warmup = c.hybrid_warmup;
    a.hybrid_threshold = c.hybrid_threshold;
    a.read_ps = c.read_ps;
    a.program_ps = c.program_ps;
    a.xfer_num = c.xfer_num;
    a.xfer_den = c.xfer_den;
    a.xfer_q = c.xfer_quantum;
    for (int k = 0; k <= 32; ++k) {
        const unsigned __int128 prod = static_cast<unsigned __int128>(1ull << k) * c.xfer_num;
        a.xfer_pow2[k] = c.xfer_quantum *
                         static_cast<std::uint64_t>((prod + c.xfer_den - 1) / c.xfer_den);
    }
    a.tile = c.tile;
    a.media_pages = c.media_pages;
    hipError_t err = halloc(e->d_pbusy, rp);
    if (err == hipSuccess) err = halloc(e->d_ptag, 2ull * rp);
    if (err == hipSuccess) err = halloc(e->d_cbusy, rc);
    if (err == hipSuccess) err = halloc(e->d_ptot, rp);
    if (err == hipSuccess) err = halloc(e->d_ctot, rc);
    if (err == hipSuccess) err = halloc(e->d_seq, 1);
    if (err == hipSuccess) err = halloc(e->d_rep, 2);
    if (err == hipSuccess) err = halloc(e->d_rep_parts, kRepParts * kRepWords);
    if (err == hipSuccess) err = halloc(e->d_disorder, 1);
    if (err == hipSuccess)
        err = hipHostMalloc(reinterpret_cast<void**>(&e->h_rep), 2 * sizeof(DevReport));
    for (int i = 0; i < 4 && err == hipSuccess; ++i) {
        err = hipEventCreate(&e->ev[i]);
    }
    if (err != hipSuccess) {
        engine_destroy(e);
        return HBFSIM_CUDA_ERROR;
    }
    const int rs = engine_reset(e);
    if (rs != HBFSIM_OK) {
        engine_destroy(e);
        return rs;
    }
    // set-up of the no-allocation entry point on this device (once per
    // device; a failed lookup only disables that entry point)
    (void)noalloc_scratch(e->device);
    *out = e;
    return HBFSIM_OK;
}

void engine_destroy(engine* e)
{
    if (e == nullptr) {
        return;
    }
    (void)hipSetDevice(e->device);
    (void)hipDeviceSynchronize();
    free_scratch(e);
    hfree(e->d_r_base);
    hfree(e->d_r_length);
    hfree(e->d_r_offset);
    hfree(e->d_r_meta);
    hfree(e->d_r_id);
    hfree(e->d_pbusy);
    hfree(e->d_ptag);
    hfree(e->d_cbusy);
    hfree(e->d_ptot);
    hfree(e->d_ctot);
    hfree(e->d_seq);
    hfree(e->d_rep);
    hfree(e->d_rep_parts);
    hfree(e->d_disorder);
    if (e->h_rep != nullptr) {
        (void)hipHostFree(e->h_rep);
    }
    for (auto& ev : e->ev) {
        if (ev != nullptr) {
            (void)hipEventDestroy(ev);
        }
    }
    delete e;
}

const engine_config& engine_get_config(const engine* e) { return e->cfg; }

int engine_set_ranges(engine* e, const std::vector<range_rec>& ranges)
{
    e->ranges = ranges;
    e->ranges_dirty = true;
    return HBFSIM_OK;
}

int engine_reset(engine* e)
{
    const std::size_t rp = e->args.Rp, rc = e->args.Rc;
    hipError_t err = hipMemset(e->d_pbusy, 0, rp * 8);
    if (err == hipSuccess) err = hipMemset(e->d_ptag, 0, rp * 16);
    if (err == hipSuccess) err = hipMemset(e->d_cbusy, 0, rc * 8);
    if (err == hipSuccess) err = hipMemset(e->d_ptot, 0, rp * 8);
    if (err == hipSuccess) err = hipMemset(e->d_ctot, 0, rc * 8);
    if (err == hipSuccess) err = hipMemset(e->d_seq, 0, 8);
    if (err == hipSuccess) err = hipMemset(e->d_disorder, 0, 4);
    if (err == hipSuccess) err = hipDeviceSynchronize();
    e->burst = 0;
    return hip_status(err);
}

int engine_synchronize(engine* e)
{
    (void)e;
    return hip_status(hipDeviceSynchronize());
}

// in_order: the records are known to be in issue order (a sorted copy), so
// the summary pass does not watch for records that go back in time.
int engine_run_any(engine* e, const void* d_rec, bool packed, std::size_t n,
                   std::uint64_t* d_comp, std::uint8_t* d_status, std::uint64_t base_ps,
                   void* stream_ptr, hbfsim_amd_report* out, bool refresh_records,
                   unsigned char* ext_scratch = nullptr, bool in_order = false);

int engine_run(engine* e, const hbf_record32* d_rec, std::size_t n, std::uint64_t* d_comp,
               std::uint8_t* d_status, std::uint64_t base_ps, void* stream_ptr,
               hbfsim_amd_report* out, bool refresh_records)
{
    return engine_run_any(e, d_rec, false, n, d_comp, d_status, base_ps, stream_ptr, out,
                          refresh_records);
}

int engine_run_packed(engine* e, const hbf_record16* d_rec, std::size_t n,
                      std::uint64_t* d_comp, std::uint8_t* d_status, std::uint64_t base_ps,
                      void* stream_ptr, hbfsim_amd_report* out)
{
    return engine_run_any(e, d_rec, true, n, d_comp, d_status, base_ps, stream_ptr, out, false);
}

int engine_run_packed_noalloc(engine* e, const hbf_record16* d_rec, std::size_t n,
                              std::uint64_t* d_comp, std::uint8_t* d_status,
                              std::uint64_t base_ps, void* stream_ptr, hbfsim_amd_report* out)
{
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    void* ptr = noalloc_scratch(e->device);
    if (ptr == nullptr) {
        return HBFSIM_UNSUPPORTED;  // the static scratch's address lookup failed
    }
    if (e->ranges_dirty) {
        return HBFSIM_UNSUPPORTED;  // uploading a changed range table allocates
    }
    return engine_run_any(e, d_rec, true, n, d_comp, d_status, base_ps, stream_ptr, out, false,
                          static_cast<unsigned char*>(ptr));
}

// Tile size of a run whose scratch comes from a fixed buffer: the engine's
// configured tile, else the automatic one doubled (up to 16,384 records)
// until the scratch fits; 0 when it never does.
std::uint32_t fitting_tile(const engine* e, std::size_t n, std::size_t capacity)
{
    KArgs a = e->args;
    std::uint32_t tile = e->cfg.tile != 0 ? e->cfg.tile : auto_tile(n);
    const std::size_t nsteps = (n + kWave - 1) / kWave;
    for (;;) {
        const std::size_t ntiles = (n + tile - 1) / tile;
        a.tile = tile;
        if (carve_scratch(a, ntiles, nsteps, nullptr, nullptr) <= capacity) {
            return tile;
        }
        if (e->cfg.tile != 0 || tile >= 16384) {
            return 0;
        }
        tile *= 2;
    }
}

int engine_run_any(engine* e, const void* d_rec, bool packed, std::size_t n,
                   std::uint64_t* d_comp, std::uint8_t* d_status, std::uint64_t base_ps,
                   void* stream_ptr, hbfsim_amd_report* out, bool refresh_records,
                   unsigned char* ext_scratch, bool in_order)
{
    if (out != nullptr) {
        std::memset(out, 0, sizeof(*out));
    }
    if (n == 0) {
        // a run of no records still uploads a changed range table, so that
        // it can prepare a context for the entry point that allocates nothing
        if (ext_scratch == nullptr && e->ranges_dirty) {
            if (hipSetDevice(e->device) != hipSuccess) {
                return HBFSIM_CUDA_ERROR;
            }
            return upload_ranges(e, static_cast<hipStream_t>(stream_ptr));
        }
        return HBFSIM_OK;
    }
    if (d_rec == nullptr || d_comp == nullptr ||
        (reinterpret_cast<std::uintptr_t>(d_rec) & 15u) != 0 ||
        (reinterpret_cast<std::uintptr_t>(d_comp) & 7u) != 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    // packed records take the main pipeline only: at most one page register,
    // the HBF model (no refresh records: they need flags); hybrid sampling
    // needs the linear steps' range ids beside their descriptors, for which
    // the run without allocation has no room
    if (packed && (e->cfg.model != HBFSIM_AMD_MODEL_HBF || e->cfg.slots > 1 ||
                   (e->cfg.hybrid != 0 && ext_scratch != nullptr))) {
        return HBFSIM_UNSUPPORTED;
    }
    if (e->cfg.model != HBFSIM_AMD_MODEL_HBF && e->cfg.model != HBFSIM_AMD_MODEL_EMPIRICAL) {
        return HBFSIM_UNSUPPORTED;
    }
    if (e->cfg.model == HBFSIM_AMD_MODEL_HBF && e->cfg.slots == 2 && refresh_records) {
        return HBFSIM_UNSUPPORTED;
    }
    // warp grouping reads group ids from 32-byte records (packed records
    // carry none); it runs on the main pipeline with at most one page
    // register and no merged refresh records
    const bool grouping = e->cfg.grouping != 0 && !packed;
    if (grouping && (e->cfg.model != HBFSIM_AMD_MODEL_HBF || e->cfg.slots == 2 ||
                     refresh_records || ext_scratch != nullptr)) {
        return HBFSIM_UNSUPPORTED;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (e->ranges_dirty) {
        const int st = upload_ranges(e, stream);
        if (st != HBFSIM_OK) {
            return st;
        }
    }
    if (e->cfg.model == HBFSIM_AMD_MODEL_EMPIRICAL) {
        if (refresh_records) {
            return HBFSIM_UNSUPPORTED;
        }
        e->last_apply_waves = 0;  // (the empirical model's own kernels, no apply pass)
        return run_empirical(e, static_cast<const hbf_record32*>(d_rec), n, d_comp, d_status,
                             base_ps, stream, out, in_order);
    }
    KArgs a = e->args;
    a.disorder = in_order ? nullptr : e->d_disorder;
    a.tile = e->cfg.tile != 0 ? e->cfg.tile : auto_tile(n);
    if (ext_scratch != nullptr) {
        a.tile = fitting_tile(e, n, kNoAllocScratchBytes);
        if (a.tile == 0) {
            return HBFSIM_UNSUPPORTED;  // beyond the static scratch
        }
    }
    const std::size_t ntiles = (n + a.tile - 1) / a.tile;
    if (ntiles > 0x7fffffffull) {
        return HBFSIM_UNSUPPORTED;
    }
    RunScratch sc{};
    int st = HBFSIM_OK;
    if (ext_scratch != nullptr) {
        (void)carve_scratch(a, ntiles, (n + kWave - 1) / kWave, ext_scratch, &sc);
    } else {
        st = ensure_scratch(e, ntiles);
        if (st != HBFSIM_OK) {
            return st;
        }
        sc = RunScratch{e->d_psum, e->d_tmask, e->d_csum, e->d_pcarry, e->d_ccarry,
                        e->d_tcount, e->d_tseq, e->d_gpsum, e->d_gcsum, e->d_gpcarry,
                        e->d_gccarry, e->d_gcount, e->d_gseq, e->d_tile_rep, nullptr,
                        e->d_tsplit};
    }
    if (packed) {
        a.tile_split = sc.tsplit;  // the summary pass marks tiles with split steps
    }
    choose_match(a);
    const std::size_t lds_a = lds_summary(a), lds_c = lds_apply(a);
    if (lds_a > kLdsPerBlockBytes || lds_c > kLdsPerBlockBytes) {
        return HBFSIM_UNSUPPORTED;
    }
    hipError_t err = hipSuccess;
    // warp grouping: mark the records that join their group's request
    // (refusing malformed groups before any state changes)
    std::uint8_t* d_lead = nullptr;
    std::uint32_t* d_gerr = nullptr;
    unsigned long long* d_frep = nullptr;
    auto free_group = [&]() {
        hfree(d_lead);
        hfree(d_gerr);
        hfree(d_frep);
    };
    if (grouping) {
        err = halloc(d_lead, n);
        if (err == hipSuccess) err = halloc(d_gerr, 1);
        if (err == hipSuccess) err = halloc(d_frep, 8);
        if (err == hipSuccess) err = hipMemsetAsync(d_gerr, 0, 4, stream);
        if (err == hipSuccess) err = hipMemsetAsync(d_frep, 0, 64, stream);
        if (err == hipSuccess) {
            const std::size_t nl = (n + kLeadSpan - 1) / kLeadSpan;
            hipLaunchKernelGGL(k_lead, dim3(static_cast<unsigned>(nl)), dim3(kWave),
                               static_cast<std::size_t>(a.r_nfence) * 8, stream, a,
                               static_cast<const hbf_record32*>(d_rec), n, d_lead, d_gerr);
            err = hipGetLastError();
        }
        std::uint32_t h_gerr = 0;
        if (err == hipSuccess)
            err = hipMemcpyAsync(&h_gerr, d_gerr, 4, hipMemcpyDeviceToHost, stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
        if (err != hipSuccess) {
            free_group();
            return HBFSIM_CUDA_ERROR;
        }
        if (h_gerr != 0) {
            free_group();
            return HBFSIM_INVALID_ARGUMENT;
        }
        a.lead = d_lead;
    }
    // two page registers: hits first, from their own scans
    const bool k2 = e->cfg.slots == 2;
    std::uint8_t* d_hits = nullptr;
    std::vector<std::uint64_t> k2_tags;
    if (k2) {
        if (halloc(d_hits, n) != hipSuccess) {
            return HBFSIM_CUDA_ERROR;
        }
        st = k2_hits(e, a, static_cast<const hbf_record32*>(d_rec), n, base_ps, ntiles, stream,
                     d_hits, k2_tags);
        if (st != HBFSIM_OK) {
            hfree(d_hits);
            return st;
        }
        a.ext_hits = 1;
    }
    // step descriptors, where the apply pass replays linear steps from them
    StepDesc* desc = nullptr;
    if (ext_scratch != nullptr) {
        desc = sc.desc;  // packed runs: one page register, no sampling; split
                         // steps go without descriptors (no side array)
    } else if ((k2 || a.slots == 1) && !grouping) {
        const std::size_t nsteps = (n + kWave - 1) / kWave;
        if (nsteps > e->desc_cap) {
            hfree(e->d_desc);
            hfree(e->d_desc_rid);
            hfree(e->d_desc_split);
            e->desc_cap = 0;
            const std::size_t cap = nsteps + nsteps / 8;  // headroom, as for the tiles
            if (halloc(e->d_desc, cap) != hipSuccess || halloc(e->d_desc_rid, cap) != hipSuccess ||
                halloc(e->d_desc_split, cap) != hipSuccess) {
                free_group();
                return HBFSIM_CUDA_ERROR;
            }
            e->desc_cap = cap;
        }
        desc = e->d_desc;
        a.desc_split = e->d_desc_split;
        if (a.hybrid != 0) {
            a.desc_rid = e->d_desc_rid;
        }
    }
    const dim3 grid(static_cast<unsigned>(ntiles));
    (void)hipEventRecord(e->ev[0], stream);
    const std::uint8_t* hits = d_hits;
    if (k2) {
        (void)allow_lds(k_summary<false, true>, lds_a);
        hipLaunchKernelGGL((k_summary<false, true>), grid, dim3(kWave), lds_a, stream, a, d_rec,
                           n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    } else if (refresh_records) {
        (void)allow_lds(k_summary<true, false>, lds_a);
        hipLaunchKernelGGL((k_summary<true, false>), grid, dim3(kWave), lds_a, stream, a, d_rec,
                           n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    } else if (packed && kLdsPerCuBytes / lds_a <= 8) {  // LDS allows at most 8 waves per CU
        (void)allow_lds(k_summary<false, false, true, true>, lds_a);
        hipLaunchKernelGGL((k_summary<false, false, true, true>), grid, dim3(kWave), lds_a, stream,
                           a, d_rec, n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    } else if (packed && ntiles <= kFewTiles) {
        (void)allow_lds(k_summary<false, false, true, false, true>, lds_a);
        hipLaunchKernelGGL((k_summary<false, false, true, false, true>), grid, dim3(kWave), lds_a,
                           stream, a, d_rec, n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    } else if (packed) {
        (void)allow_lds(k_summary<false, false, true>, lds_a);
        hipLaunchKernelGGL((k_summary<false, false, true>), grid, dim3(kWave), lds_a, stream, a,
                           d_rec, n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    } else {
        (void)allow_lds(k_summary<false, false>, lds_a);
        hipLaunchKernelGGL((k_summary<false, false>), grid, dim3(kWave), lds_a, stream, a, d_rec,
                           n, base_ps, sc.psum, sc.tmask, sc.csum, sc.tcount,
                           hits, desc);
    }
    (void)hipEventRecord(e->ev[1], stream);
    {
        const std::size_t ngroups = (ntiles + kGroup - 1) / kGroup;
        const std::size_t rt = static_cast<std::size_t>(a.Rp) + a.Rc + 1;
        const unsigned wide = static_cast<unsigned>((ngroups * rt + 255) / 256);
        if (ntiles <= kOneCarryTiles) {
            const auto span = static_cast<std::uint32_t>((ntiles + kMidBlock - 1) / kMidBlock);
            hipLaunchKernelGGL(k_carry_one, dim3(static_cast<unsigned>(rt)), dim3(kMidBlock), 0,
                               stream, a, ntiles, span, sc.psum, sc.tmask, sc.csum,
                               sc.tcount, sc.pcarry, sc.ccarry, sc.tseq, e->d_pbusy, e->d_ptag,
                               e->d_cbusy, e->d_seq, e->d_ptot, e->d_ctot);
        } else {
            hipLaunchKernelGGL(k_carry_up, dim3(wide), dim3(256), 0, stream, a, ntiles, ngroups,
                               sc.psum, sc.tmask, sc.csum, sc.tcount, sc.gpsum,
                               sc.gcsum, sc.gcount);
            hipLaunchKernelGGL(k_carry_mid, dim3(a.Rp + a.Rc + 1), dim3(kMidBlock), 0, stream, a,
                               ngroups,
                               sc.gpsum, sc.gcsum, sc.gcount, sc.gpcarry, sc.gccarry,
                               sc.gseq, e->d_pbusy, e->d_ptag, e->d_cbusy, e->d_seq, e->d_ptot,
                               e->d_ctot);
            hipLaunchKernelGGL(k_carry_down, dim3(wide), dim3(256), 0, stream, a, ntiles, ngroups,
                               sc.psum, sc.tmask, sc.csum, sc.tcount, sc.gpcarry,
                               sc.gccarry, sc.gseq, sc.pcarry, sc.ccarry, sc.tseq);
        }
    }
    (void)hipEventRecord(e->ev[2], stream);
    const bool staged = desc != nullptr && staged_steps(a) != 0;
    // the four-wave apply pass: a large stream whose last run on this engine
    // had few page-register hits (mostly general steps), where LDS leaves
    // room for four waves per SIMD
    const bool wide_apply = packed && n >= kWideApplyRecords &&
                            kLdsPerCuBytes / lds_c >= 4 * kSimdsPerCu && e->last_modeled != 0 &&
                            e->last_hits * 8 < e->last_modeled;
    e->last_apply_waves = packed && !k2 && !refresh_records ? (wide_apply ? 4 : 3) : 1;
    if (k2) {
        (void)allow_lds(k_apply<false, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, true>), grid, dim3(kWave), lds_c, stream, a, d_rec, n,
                           base_ps, sc.pcarry, sc.tmask, sc.ccarry, sc.tseq, d_comp,
                           d_status, sc.tile_rep, hits, desc);
    } else if (refresh_records && staged) {
        (void)allow_lds(k_apply<true, false, true>, lds_c);
        hipLaunchKernelGGL((k_apply<true, false, true>), grid, dim3(kWave), lds_c, stream, a,
                           d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry, sc.tseq,
                           d_comp, d_status, sc.tile_rep, hits, desc);
    } else if (refresh_records) {
        (void)allow_lds(k_apply<true, false>, lds_c);
        hipLaunchKernelGGL((k_apply<true, false>), grid, dim3(kWave), lds_c, stream, a, d_rec, n,
                           base_ps, sc.pcarry, sc.tmask, sc.ccarry, sc.tseq, d_comp,
                           d_status, sc.tile_rep, hits, desc);
    } else if (packed && staged && wide_apply) {
        (void)allow_lds(k_apply<false, false, true, true, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false, true, true, true>), grid, dim3(kWave), lds_c,
                           stream, a, d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry,
                           sc.tseq, d_comp, d_status, sc.tile_rep, hits, desc);
    } else if (packed && staged) {
        (void)allow_lds(k_apply<false, false, true, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false, true, true>), grid, dim3(kWave), lds_c, stream,
                           a, d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry,
                           sc.tseq, d_comp, d_status, sc.tile_rep, hits, desc);
    } else if (packed && wide_apply) {
        (void)allow_lds(k_apply<false, false, false, true, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false, false, true, true>), grid, dim3(kWave), lds_c,
                           stream, a, d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry,
                           sc.tseq, d_comp, d_status, sc.tile_rep, hits, desc);
    } else if (packed) {
        (void)allow_lds(k_apply<false, false, false, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false, false, true>), grid, dim3(kWave), lds_c, stream,
                           a, d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry,
                           sc.tseq, d_comp, d_status, sc.tile_rep, hits, desc);
    } else if (staged) {
        (void)allow_lds(k_apply<false, false, true>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false, true>), grid, dim3(kWave), lds_c, stream, a,
                           d_rec, n, base_ps, sc.pcarry, sc.tmask, sc.ccarry, sc.tseq,
                           d_comp, d_status, sc.tile_rep, hits, desc);
    } else {
        (void)allow_lds(k_apply<false, false>, lds_c);
        hipLaunchKernelGGL((k_apply<false, false>), grid, dim3(kWave), lds_c, stream, a, d_rec, n,
                           base_ps, sc.pcarry, sc.tmask, sc.ccarry, sc.tseq, d_comp,
                           d_status, sc.tile_rep, hits, desc);
    }
    // (the apply pass's interval ends with it: the report reduction's two
    // small launches are no part of it)
    (void)hipEventRecord(e->ev[3], stream);
    launch_report(stream, sc.tile_rep, ntiles, e->d_rep, e->d_rep_parts, e->d_disorder);
    unsigned long long h_frep[8] = {};
    if (grouping) {
        const std::size_t nb = (n + 255) / 256;
        hipLaunchKernelGGL(k_follow,
                           dim3(static_cast<unsigned>(nb < kFollowBlocks ? nb : kFollowBlocks)),
                           dim3(256), 0, stream, static_cast<const hbf_record32*>(d_rec), n,
                           base_ps, d_lead, d_comp, d_status, d_frep);
    }
    err = hipGetLastError();
    if (err == hipSuccess)
        err = hipMemcpyAsync(e->h_rep, e->d_rep, sizeof(DevReport) + 8, hipMemcpyDeviceToHost,
                             stream);
    if (err == hipSuccess && grouping)
        err = hipMemcpyAsync(h_frep, d_frep, sizeof(h_frep), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    const bool went_back = err == hipSuccess && e->h_rep[1].v[0] != 0;
    // two page registers: the tags the run leaves, unless it is timed again
    if (err == hipSuccess && k2 && !went_back) {
        err = hipMemcpyAsync(e->d_ptag, k2_tags.data(), k2_tags.size() * 8, hipMemcpyHostToDevice,
                             stream);
        if (err == hipSuccess) err = hipStreamSynchronize(stream);
    }
    hfree(d_hits);
    free_group();
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (went_back) {
        // Some record's issue time went back: the engine state is as the run
        // found it.  The stream is served in (issue time, position) order,
        // from a sorted copy, which the entry point without allocation
        // cannot make.
        if (ext_scratch != nullptr) {
            return HBFSIM_INVALID_ARGUMENT;
        }
        return run_in_issue_order(
            d_rec, packed, n, d_comp, d_status, stream_ptr,
            [&](const void* sorted, std::uint64_t* comp, std::uint8_t* status) {
                return engine_run_any(e, sorted, packed, n, comp, status, base_ps, stream_ptr,
                                      out, refresh_records, nullptr, true);
            });
    }
    e->last_modeled = e->h_rep[0].v[R_MODELED];
    e->last_hits = e->h_rep[0].v[R_HITS];
    for (int k = 0; k < 3; ++k) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e->ev[k], e->ev[k + 1]) == hipSuccess) {
            e->last_ms[k] = ms;
        }
    }
    if (out != nullptr) {
        std::memcpy(out, e->h_rep, sizeof(DevReport));
        if (grouping) {
            // the joined records: modeled, read or write, their latencies
            out->grouped = h_frep[0];
            out->modeled += h_frep[0];
            out->reads += h_frep[1];
            out->writes += h_frep[2];
            out->makespan_ps = std::max<std::uint64_t>(out->makespan_ps, h_frep[3]);
            const std::uint64_t lo = out->latency_sum_lo + h_frep[4];
            out->latency_sum_hi += h_frep[5] + (lo < out->latency_sum_lo ? 1u : 0u);
            out->latency_sum_lo = lo;
            out->latency_max_ps = std::max<std::uint64_t>(out->latency_max_ps, h_frep[6]);
        }
    }
    return HBFSIM_OK;
}

int engine_run_host(engine* e, const hbf_record32* records, std::size_t n,
                    std::uint64_t* completion, std::uint8_t* status, std::uint64_t base_ps,
                    hbfsim_amd_report* out)
{
    if (out != nullptr) {
        std::memset(out, 0, sizeof(*out));
    }
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (records == nullptr || completion == nullptr) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    hbf_record32* d_rec = nullptr;
    std::uint64_t* d_comp = nullptr;
    std::uint8_t* d_st = nullptr;
    hipError_t err = halloc(d_rec, n);
    if (err == hipSuccess) err = halloc(d_comp, n);
    if (err == hipSuccess && status != nullptr) err = halloc(d_st, n);
    if (err == hipSuccess)
        err = hipMemcpy(d_rec, records, n * sizeof(hbf_record32), hipMemcpyHostToDevice);
    int st = hip_status(err);
    if (st == HBFSIM_OK) {
        st = engine_run(e, d_rec, n, d_comp, d_st, base_ps, nullptr, out);
    }
    if (st == HBFSIM_OK) {
        err = hipMemcpy(completion, d_comp, n * 8, hipMemcpyDeviceToHost);
        if (err == hipSuccess && status != nullptr)
            err = hipMemcpy(status, d_st, n, hipMemcpyDeviceToHost);
        st = hip_status(err);
    }
    hfree(d_rec);
    hfree(d_comp);
    hfree(d_st);
    return st;
}

int engine_get_busy_totals(engine* e, std::uint64_t* plane_ps, std::size_t planes,
                           std::uint64_t* channel_ps, std::size_t channels)
{
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (plane_ps != nullptr) {
        if (planes < e->args.Rp) return HBFSIM_INVALID_ARGUMENT;
        if (hipMemcpy(plane_ps, e->d_ptot, e->args.Rp * 8ull, hipMemcpyDeviceToHost) != hipSuccess)
            return HBFSIM_CUDA_ERROR;
    }
    if (channel_ps != nullptr) {
        if (channels < e->args.Rc) return HBFSIM_INVALID_ARGUMENT;
        if (hipMemcpy(channel_ps, e->d_ctot, e->args.Rc * 8ull, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return HBFSIM_CUDA_ERROR;
    }
    return HBFSIM_OK;
}

int engine_get_state(engine* e, std::uint64_t* plane_busy, std::uint64_t* plane_tags,
                     std::uint64_t* channel_cursor, std::uint64_t* sequence, std::uint64_t* burst)
{
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    const std::size_t rp = e->args.Rp, rc = e->args.Rc;
    hipError_t err = hipSuccess;
    if (plane_busy) err = hipMemcpy(plane_busy, e->d_pbusy, rp * 8, hipMemcpyDeviceToHost);
    if (err == hipSuccess && plane_tags)
        err = hipMemcpy(plane_tags, e->d_ptag, rp * 16, hipMemcpyDeviceToHost);
    if (err == hipSuccess && channel_cursor)
        err = hipMemcpy(channel_cursor, e->d_cbusy, rc * 8, hipMemcpyDeviceToHost);
    if (err == hipSuccess && sequence)
        err = hipMemcpy(sequence, e->d_seq, 8, hipMemcpyDeviceToHost);
    if (burst) *burst = e->burst;
    return hip_status(err);
}

int engine_set_state(engine* e, const std::uint64_t* plane_busy, const std::uint64_t* plane_tags,
                     const std::uint64_t* channel_cursor, std::uint64_t sequence,
                     std::uint64_t burst)
{
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    const std::size_t rp = e->args.Rp, rc = e->args.Rc;
    hipError_t err = hipSuccess;
    if (plane_busy) err = hipMemcpy(e->d_pbusy, plane_busy, rp * 8, hipMemcpyHostToDevice);
    if (err == hipSuccess && plane_tags)
        err = hipMemcpy(e->d_ptag, plane_tags, rp * 16, hipMemcpyHostToDevice);
    if (err == hipSuccess && channel_cursor)
        err = hipMemcpy(e->d_cbusy, channel_cursor, rc * 8, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(e->d_seq, &sequence, 8, hipMemcpyHostToDevice);
    e->burst = burst;
    return hip_status(err);
}

int engine_last_kernel_ms(const engine* e, float* ms, int max_kernels)
{
    const int k = std::min(3, max_kernels);
    for (int i = 0; i < k; ++i) {
        ms[i] = e->last_ms[i];
    }
    return k;
}

int engine_last_apply_waves(const engine* e)
{
    return e->last_apply_waves;
}


int engine_window_counts(engine* e, const hbf_record32* d_rec, std::size_t n,
                         std::uint64_t window_ps, std::uint64_t windows, std::uint32_t* d_counts,
                         void* stream_ptr)
{
    if (n == 0) {
        return HBFSIM_OK;
    }
    if (d_rec == nullptr || d_counts == nullptr || window_ps == 0 ||
        (reinterpret_cast<std::uintptr_t>(d_rec) & 15u) != 0) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (hipSetDevice(e->device) != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (e->ranges_dirty) {
        const int st = upload_ranges(e, stream);
        if (st != HBFSIM_OK) {
            return st;
        }
    }
    const KArgs& a = e->args;
    const std::uint32_t ndie = a.Rp / a.P;
    const std::size_t lds = 8ull * a.r_nfence + 4ull * kCountBins;
    const std::size_t blocks = (n + kCountChunk - 1) / kCountChunk;
    hipLaunchKernelGGL(k_window_counts, dim3(static_cast<unsigned>(blocks)), dim3(256), lds, stream,
                       a, d_rec, n, window_ps, windows, ndie, d_counts);
    return hip_status(hipGetLastError());
}

}  // namespace hbfamd
