// link.hip -- the UCIe Streaming / AoU link (src/ucie/link.cpp:1-203) for
// batches of independent links on gfx950 (MI355X).
//
// Two lanes run one link's event loop, one per direction: AR requests (3
// AoU granules) and R returns (14) queue per direction; a direction sends a Format 6 flit of 48
// granules every 32 / GT ns while it has work; a message's granules are all
// reserved against the sender's credits at its MsgStart; a delivered message
// is consumed a fixed delay later by the link's caller, which releases its
// credits as a grant that rides the next flit of the other direction in the
// legal AoU amounts (1, 4, 8, ... 128).  Messages of a direction move through
// the link in order, so every event source of a direction is a FIFO: the
// admitted messages (arrivals), the in-flight flits (deliveries), the
// delivered messages (consumes), plus the serializer's free time (retry).
// The loop needs no priority queue: the next event is the least of at most
// eight FIFO heads and two retry times, and the caller's FIFO admission
// (at most max_accepted messages in flight per direction) is a counter.
// A split pass first lays each link's messages out as two lists, AR then R,
// so that every FIFO cursor is a counter and the next admission's ready time
// is fetched one message ahead instead of by a dependent scan of the
// direction bytes.
//
// Events at one time are taken as the reference's step() takes them: every
// arrival, delivery and consume already scheduled at that time, then both
// directions send.  A consume scheduled by this step's deliveries is taken
// by the next step, even at the same time, as the reference's caller
// schedules it after step() returns.
#include <hip/hip_runtime.h>

#include "link.hpp"

#include <cstring>
#include <mutex>

namespace hbfamd {
namespace {

constexpr int kLinkThreads = 64;
constexpr int kSplitWaves = 4;  // links per workgroup of the split pass
constexpr std::uint64_t kBadLink = ~0ull;

struct LinkArgs {
    std::uint64_t ser, prop;
    std::uint64_t delay[2];
    std::uint32_t credit0[2];      // initial sender credits: [0] AR, [1] R
    std::uint32_t max_accepted;
    std::uint32_t ring;            // in-flight flit slots per direction
    std::uint32_t links;
    std::uint64_t n;               // messages in all links
    const std::uint64_t* first;    // [links + 1]
    const std::uint64_t* ready;
    const std::uint8_t* dir;
    std::uint64_t* delivered;
    std::uint64_t* counters;       // [links][2][9]
    hbfsim_amd_link_flit* trace;   // [links][2][trace_limit] (kTrace launches)
    std::uint32_t trace_limit;
    // the split pass's output: each link's messages at [first, first[l+1]),
    // its AR messages first, then its R messages, each in arrival order
    std::uint64_t* part_time;      // ready time (HBM form: then admission, delivery time)
    std::uint32_t* part_index;     // message index within the link
    std::uint64_t* n_ar;           // [links]: AR messages, or kBadLink
    std::uint64_t* ring_time;      // HBM form: [links][2][ring]
    std::uint32_t* ring_info;      // HBM form: [links][2][ring]: grant << 16 | completed
    std::uint32_t* error;          // 1 overflow or bad input, 2 iteration cap
};

__device__ __forceinline__ std::uint32_t legal_grant(std::uint32_t pending)
{
    if (pending == 0) {
        return 0;
    }
    if (pending < 4) {
        return 1;
    }
    std::uint32_t g = 4;
    while (g < 128 && g * 2 <= pending) {
        g *= 2;
    }
    return g;
}

// One wave per link: count the link's AR messages (ballots), then scatter
// every message to its rank within its direction's list.  Directions other
// than 0 and 1 and malformed offsets mark the link bad.
__global__ __launch_bounds__(kSplitWaves * 64) void k_link_split(LinkArgs a)
{
    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t l = blockIdx.x * kSplitWaves + (threadIdx.x >> 6);
    if (l >= a.links) {
        return;
    }
    const std::uint64_t b = a.first[l], e = a.first[l + 1];
    if (b > e || e > a.n || e - b > 0xffffffffull) {
        if (lane == 0) {
            a.n_ar[l] = kBadLink;
            atomicMax(a.error, 1u);
        }
        return;
    }
    const std::uint64_t below = (1ull << lane) - 1;
    std::uint64_t ar = 0;
    bool bad = false;
    for (std::uint64_t base = b; base < e; base += 64) {
        const std::uint64_t i = base + lane;
        const std::uint32_t d = i < e ? a.dir[i] : 0u;
        bad = bad || d > 1;
        ar += __popcll(__ballot(i < e && d == 0));
    }
    if (__ballot(bad) != 0) {
        if (lane == 0) {
            a.n_ar[l] = kBadLink;
            atomicMax(a.error, 1u);
        }
        return;
    }
    std::uint64_t c0 = b, c1 = b + ar;
    for (std::uint64_t base = b; base < e; base += 64) {
        const std::uint64_t i = base + lane;
        const bool live = i < e;
        const std::uint32_t d = live ? a.dir[i] : 0u;
        const std::uint64_t m0 = __ballot(live && d == 0), m1 = __ballot(live && d == 1);
        if (live) {
            const std::uint64_t pos = d == 0 ? c0 + __popcll(m0 & below) : c1 + __popcll(m1 & below);
            a.part_time[pos] = a.ready[i];
            a.part_index[pos] = static_cast<std::uint32_t>(i - b);
        }
        c0 += __popcll(m0);
        c1 += __popcll(m1);
    }
    if (lane == 0) {
        a.n_ar[l] = ar;
    }
}

// The message FIFOs and in-flight flit rings of a link live either in LDS
// (the fast forms: at most kMsg messages admitted per direction and kFlit
// flits in flight) or in HBM: the message times in place of their ready
// times in the split lists, the flit rings in a scratch buffer.  The small
// form (4 + 4 slots, 6 KiB per 64-lane workgroup) serves the reference's
// default of 4 admitted messages without propagation delay and leaves room
// for 6 waves per SIMD; the large one (16 + 8, 18 KiB: 2 waves per SIMD)
// serves up to 16 admitted messages and propagation up to 5 flit times.
constexpr std::uint32_t kSmallMsg = 4, kSmallFlit = 4;
constexpr std::uint32_t kLargeMsg = 16, kLargeFlit = 8;

// The partner lane's value (lane ^ 1: the same link's other direction), by
// DPP quad_perm [1, 0, 3, 2].  Both lanes of a link run the loop in step.
__device__ __forceinline__ std::uint32_t pair32(std::uint32_t v)
{
    return static_cast<std::uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));
}

__device__ __forceinline__ std::uint64_t pair64(std::uint64_t v)
{
    return (static_cast<std::uint64_t>(pair32(static_cast<std::uint32_t>(v >> 32))) << 32) |
           pair32(static_cast<std::uint32_t>(v));
}

// Two lanes per link, one per direction (lane & 1: 0 AR, 1 R).  The
// directions meet only through the event time, the grants a delivered flit
// carries to the other direction's credits, the consumes that fill the
// other direction's pending grant, and errors: those cross between the two
// lanes once per step, at the points where the reference's step() would
// read them, and everything else is the lane's own direction.
// kTrace: also record each direction's first trace_limit flits with their
// fragments (the head message's identity comes from its FIFO slot).
template <std::uint32_t kMsg, std::uint32_t kFlit, bool kTrace = false>
__global__ __launch_bounds__(kLinkThreads) void k_link(LinkArgs a)
{
    constexpr bool kLds = kMsg != 0;  // else the HBM form
    __shared__ std::uint64_t s_msg_t[kLds ? kMsg * kLinkThreads : 1];
    __shared__ std::uint32_t s_msg_i[kLds ? kMsg * kLinkThreads : 1];
    __shared__ std::uint64_t s_fl_t[kLds ? kFlit * kLinkThreads : 1];
    __shared__ std::uint32_t s_fl_i[kLds ? kFlit * kLinkThreads : 1];
    const std::uint32_t lane = threadIdx.x;
    const std::uint32_t d = lane & 1u;
    const std::uint32_t l = blockIdx.x * (kLinkThreads / 2) + (lane >> 1);
    if (l >= a.links) {
        return;  // both lanes of the link
    }
    const std::uint64_t ar = a.n_ar[l];
    if (ar == kBadLink) {
        return;  // refused by the split pass
    }
    const std::uint64_t b = a.first[l], e = a.first[l + 1];
    const std::uint64_t base = d == 0 ? b : b + ar;  // this direction's list
    // the split pass refuses links of 2^32 messages or more
    const std::uint32_t count = static_cast<std::uint32_t>(d == 0 ? ar : e - b - ar);
    const std::uint32_t size = d == 0 ? 3u : 14u;    // granules of this direction's messages
    const std::uint32_t osize = d == 0 ? 14u : 3u;   // and of the other's
    const std::uint64_t delay = a.delay[d];
    const std::uint32_t credit0 = a.credit0[d];
    const std::uint32_t M = a.max_accepted;
    // flit slot s: LDS lane-minor (conflict-free), HBM link-major
    auto fl_t = [&](std::uint32_t s) -> std::uint64_t& {
        if constexpr (kLds) {
            return s_fl_t[s * kLinkThreads + lane];
        } else {
            return a.ring_time[(2ull * l + d) * a.ring + s];
        }
    };
    auto fl_i = [&](std::uint32_t s) -> std::uint32_t& {
        if constexpr (kLds) {
            return s_fl_i[s * kLinkThreads + lane];
        } else {
            return a.ring_info[(2ull * l + d) * a.ring + s];
        }
    };
    // message k (LDS slot s = k mod max_accepted)
    auto msg_t = [&](std::uint32_t k, std::uint32_t s) -> std::uint64_t& {
        if constexpr (kLds) {
            return s_msg_t[s * kLinkThreads + lane];
        } else {
            return a.part_time[base + k];
        }
    };
    auto msg_i = [&](std::uint32_t k, std::uint32_t s) -> std::uint32_t {
        if constexpr (kLds) {
            return s_msg_i[s * kLinkThreads + lane];
        } else {
            return a.part_index[base + k];
        }
    };
    auto wrap = [&](std::uint32_t s) -> std::uint32_t { return s + 1 == M ? 0u : s + 1; };
    // messages admitted, arrived, sent, delivered, consumed, with their LDS
    // slots; the next admission's ready time and index
    std::uint32_t n_adm = 0, n_arr = 0, n_done = 0, n_dlv = 0, n_con = 0;
    std::uint32_t s_adm = 0, s_arr = 0, s_dlv = 0, s_con = 0;
    std::uint32_t s_done = 0;  // (kTrace) the slot of the message being sent
    std::uint64_t next_ready = 0, last_ready = 0;
    std::uint32_t next_index = 0;
    std::uint32_t h_rem = size, h_started = 0;
    std::uint64_t cursor = 0;
    std::uint32_t credits = credit0;
    std::uint32_t gp = 0;  // credits to grant back on this direction's flits
    std::uint32_t rh = 0, rn = 0;  // flit ring head, entries
    std::uint64_t flits = 0, gran = 0, credit_only = 0;
    if (count != 0) {
        next_ready = a.part_time[base];
        next_index = kLds ? a.part_index[base] : 0u;
    }
    std::uint64_t now = 0;
    std::uint32_t err = 0;
    const std::uint64_t cap = 64ull * (e - b) + 4096;
    for (std::uint64_t it = 0;; ++it) {
        if (it >= cap) {
            err = 2;
            break;
        }
        // the caller admits waiting messages while the direction has room
        while (n_adm < count && n_adm - n_con < M) {
            const std::uint64_t r = next_ready;
            if (r < last_ready) {
                err = 1;  // a direction's ready times must not decrease
            }
            last_ready = r;
            msg_t(n_adm, s_adm) = r > now ? r : now;
            if constexpr (kLds) {
                s_msg_i[s_adm * kLinkThreads + lane] = next_index;
                s_adm = wrap(s_adm);
            }
            ++n_adm;
            if (n_adm < count) {  // fetch the next admission ahead of its use
                next_ready = a.part_time[base + n_adm];
                if constexpr (kLds) {
                    next_index = a.part_index[base + n_adm];
                }
            }
        }
        if ((err | pair32(err)) != 0) {
            break;
        }
        // the next event: the least over both directions
        bool any = false;
        std::uint64_t t = ~0ull;
        if (n_arr < n_adm) {
            const std::uint64_t x = msg_t(n_arr, s_arr);
            t = x < t ? x : t;
            any = true;
        }
        if (rn != 0) {
            const std::uint64_t x = fl_t(rh);
            t = x < t ? x : t;
            any = true;
        }
        if (n_con < n_dlv) {
            const std::uint64_t dv = msg_t(n_con, s_con);
            if (dv > ~0ull - delay) {
                err = 1;
            }
            const std::uint64_t x = dv + delay;
            t = x < t ? x : t;
            any = true;
        }
        if (cursor > now && (n_arr > n_done || gp != 0)) {
            t = cursor < t ? cursor : t;
            any = true;
        }
        const std::uint64_t tp = pair64(t);
        const std::uint32_t anyp = pair32(any ? 1u : 0u);
        if ((err | pair32(err)) != 0 || (!any && anyp == 0)) {
            break;
        }
        now = t < tp ? t : tp;
        // every arrival, delivery and consume scheduled at `now`; consumes
        // of messages this step delivers wait for the next step
        const std::uint32_t dlv_before = n_dlv;
        while (n_arr < n_adm && msg_t(n_arr, s_arr) == now) {
            ++n_arr;
            s_arr = wrap(s_arr);
        }
        std::uint32_t g_out = 0;  // the grant this direction's flit brings the other
        if (rn != 0 && fl_t(rh) == now) {
            const std::uint32_t info = fl_i(rh);
            const std::uint32_t done = info & 0xffffu;
            g_out = info >> 16;
            for (std::uint32_t k = 0; k < done; ++k) {
                msg_t(n_dlv, s_dlv) = now;
                a.delivered[b + msg_i(n_dlv, s_dlv)] = now;
                ++n_dlv;
                s_dlv = wrap(s_dlv);
            }
            rh = rh + 1 == a.ring ? 0u : rh + 1;
            --rn;
        }
        std::uint32_t c_out = 0;  // consumes, each a grant of `size` for the other
        while (n_con < dlv_before && msg_t(n_con, s_con) + delay == now) {
            ++c_out;
            ++n_con;
            s_con = wrap(s_con);
        }
        const std::uint32_t g_in = pair32(g_out);
        const std::uint32_t c_in = pair32(c_out);
        if (g_in > credit0 - credits) {
            err = 1;
        }
        credits += g_in;
        if (static_cast<std::uint64_t>(gp) + static_cast<std::uint64_t>(c_in) * osize > 65535u) {
            err = 1;
        } else {
            gp += c_in * osize;
        }
        if ((err | pair32(err)) != 0) {
            break;
        }
        // this direction sends (link.cpp send_ready)
        if (cursor <= now) {
            std::uint32_t used = 0, done = 0, nfrag = 0;
            hbfsim_amd_link_flit* rec = nullptr;
            if constexpr (kTrace) {
                if (flits < a.trace_limit) {
                    rec = a.trace + (2ull * l + d) * a.trace_limit + flits;
                }
            }
            while (n_arr > n_done && used < 48) {
                if (!h_started) {
                    if (credits < size) {
                        break;
                    }
                    credits -= size;
                    h_started = 1;
                }
                const std::uint32_t frag = 48 - used < h_rem ? 48 - used : h_rem;
                if constexpr (kTrace) {
                    if (rec != nullptr) {  // link.cpp:115-119
                        hbfsim_amd_link_fragment f;
                        f.request_id = static_cast<std::uint64_t>(msg_i(n_done, s_done)) + 1;
                        f.flit_granule = used;
                        f.message_granule = size - h_rem;
                        f.granules = frag;
                        f.msg_start = h_rem == size ? 1 : 0;
                        f.msg_end = frag == h_rem ? 1 : 0;
                        f.reserved[0] = f.reserved[1] = 0;
                        rec->fragment[nfrag] = f;
                    }
                }
                ++nfrag;
                used += frag;
                h_rem -= frag;
                if (h_rem == 0) {
                    ++done;
                    ++n_done;
                    s_done = kLds ? wrap(s_done) : 0u;
                    h_rem = size;
                    h_started = 0;
                }
            }
            const std::uint32_t grant = legal_grant(gp);
            if (used != 0 || grant != 0) {
                gp -= grant;
                if (now > ~0ull - a.ser || now + a.ser > ~0ull - a.prop || rn == a.ring) {
                    err = 1;
                } else {
                    cursor = now + a.ser;
                    const std::uint32_t slot = rh + rn < a.ring ? rh + rn : rh + rn - a.ring;
                    fl_t(slot) = cursor + a.prop;
                    fl_i(slot) = (grant << 16) | done;
                    if constexpr (kTrace) {
                        if (rec != nullptr) {  // link.cpp:150-156
                            rec->start_ns = now;
                            rec->delivered_ns = cursor + a.prop;
                            rec->step = it;
                            rec->direction = d;
                            rec->message_granules = used;
                            rec->grant_granules = grant;
                            rec->credit_only = used == 0 ? 1u : 0u;
                            rec->fragments = nfrag;
                            rec->reserved = 0;
                        }
                    }
                    ++rn;
                    ++flits;
                    gran += used;
                    credit_only += used == 0 ? 1u : 0u;
                }
            }
        }
        if ((err | pair32(err)) != 0) {
            break;
        }
    }
    if (err != 0) {
        atomicMax(a.error, err);
    }
    // the reference adds per flit, each count bounded at 2^64 - 1
    // (link.cpp:15-23, 140-149); in closed form a count of k per flit is
    // bounded iff its total exceeds the bound
    std::uint64_t* c = a.counters + (2ull * l + d) * 9;
    bool sat = false;
    const auto bounded = [&](std::uint64_t per, std::uint64_t times) -> std::uint64_t {
        if (times != 0 && per > ~0ull / times) {
            sat = true;
            return ~0ull;
        }
        return per * times;
    };
    c[0] = flits;
    c[1] = bounded(256, flits);
    c[2] = bounded(2, flits);
    c[3] = bounded(4, flits);
    c[4] = bounded(10, flits);
    c[5] = bounded(5, gran);
    c[6] = bounded(5, 48 * flits - gran);
    c[7] = credit_only;
    c[8] = sat ? 1u : 0u;
}

// The split lists and flit rings of the last, largest call, kept per device
// (grown on demand, held until the process ends); a call holds its device's
// lock until it has synchronised, so calls on one device run one at a time.
struct LinkScratch {
    std::mutex mu;
    unsigned char* ptr = nullptr;
    std::size_t bytes = 0;
};
constexpr int kMaxDevices = 64;
LinkScratch g_scratch[kMaxDevices];

}  // namespace

int link_run(const hbfsim_amd_link_profile& p, const std::uint64_t* d_first, std::uint32_t links,
             const std::uint64_t* d_ready, const std::uint8_t* d_dir, std::size_t n,
             std::uint64_t* d_delivered, hbfsim_amd_link_counters* d_counters, void* stream_ptr,
             hbfsim_amd_link_flit* d_flits, std::uint32_t flit_limit)
{
    if (p.gt_per_second != 8 && p.gt_per_second != 16 && p.gt_per_second != 32) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (p.initial_ar_granules < 3 || p.initial_r_granules < 14 ||
        p.initial_ar_granules > 65535 || p.initial_r_granules > 65535 || p.max_accepted == 0 ||
        p.max_accepted > 65535 || p.propagation_ns > 1000000000ull) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    if (links == 0) {
        return HBFSIM_OK;
    }
    if (d_first == nullptr || d_counters == nullptr ||
        (n != 0 && (d_ready == nullptr || d_dir == nullptr || d_delivered == nullptr))) {
        return HBFSIM_INVALID_ARGUMENT;
    }
    const std::uint64_t ser = 32u / p.gt_per_second;
    // flits in flight per direction: one leaves every ser ns and arrives
    // ser + propagation later
    const std::uint64_t ring = (ser + p.propagation_ns) / ser + 2;
    if (ring > 4096) {
        return HBFSIM_UNSUPPORTED;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const bool small = p.max_accepted <= kSmallMsg && ring <= kSmallFlit;
    const bool lds = small || (p.max_accepted <= kLargeMsg && ring <= kLargeFlit);
    // one allocation: the split lists, the AR counts, the flit rings (HBM
    // form) and the error flag, each piece 256-byte aligned
    auto up = [](std::size_t x) { return (x + 255) & ~std::size_t{255}; };
    const std::size_t nn = n == 0 ? 1 : n;
    const std::size_t o_time = 0, o_index = o_time + up(nn * 8), o_ar = o_index + up(nn * 4);
    const std::size_t o_rt = o_ar + up(std::size_t{links} * 8);
    const std::size_t o_ri = o_rt + (lds ? 0 : up(2ull * links * ring * 8));
    const std::size_t o_err = o_ri + (lds ? 0 : up(2ull * links * ring * 4));
    const std::size_t bytes = o_err + 256;
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    if (device < 0 || device >= kMaxDevices) {
        return HBFSIM_UNSUPPORTED;
    }
    LinkScratch& cache = g_scratch[device];
    std::lock_guard<std::mutex> hold(cache.mu);
    if (cache.bytes < bytes) {
        if (cache.ptr != nullptr) {
            (void)hipFree(cache.ptr);
            cache.ptr = nullptr;
            cache.bytes = 0;
        }
        err = hipMalloc(reinterpret_cast<void**>(&cache.ptr), bytes);
        if (err != hipSuccess) {
            cache.ptr = nullptr;
            return HBFSIM_CUDA_ERROR;
        }
        cache.bytes = bytes;
    }
    unsigned char* scratch = cache.ptr;
    std::uint32_t h_err = 0;
    if (err == hipSuccess) err = hipMemsetAsync(scratch + o_err, 0, 4, stream);
    if (err == hipSuccess) {
        LinkArgs a;
        std::memset(&a, 0, sizeof(a));
        a.ser = ser;
        a.prop = p.propagation_ns;
        a.delay[0] = p.consume_delay_ns[0];
        a.delay[1] = p.consume_delay_ns[1];
        a.credit0[0] = p.initial_ar_granules;
        a.credit0[1] = p.initial_r_granules;
        a.max_accepted = p.max_accepted;
        a.ring = static_cast<std::uint32_t>(ring);
        a.links = links;
        a.n = n;
        a.first = d_first;
        a.ready = d_ready;
        a.dir = d_dir;
        a.delivered = d_delivered;
        a.counters = reinterpret_cast<std::uint64_t*>(d_counters);
        a.trace = d_flits;
        a.trace_limit = flit_limit;
        a.part_time = reinterpret_cast<std::uint64_t*>(scratch + o_time);
        a.part_index = reinterpret_cast<std::uint32_t*>(scratch + o_index);
        a.n_ar = reinterpret_cast<std::uint64_t*>(scratch + o_ar);
        a.ring_time = lds ? nullptr : reinterpret_cast<std::uint64_t*>(scratch + o_rt);
        a.ring_info = lds ? nullptr : reinterpret_cast<std::uint32_t*>(scratch + o_ri);
        a.error = reinterpret_cast<std::uint32_t*>(scratch + o_err);
        hipLaunchKernelGGL(k_link_split, dim3((links + kSplitWaves - 1) / kSplitWaves),
                           dim3(kSplitWaves * 64), 0, stream, a);
        err = hipGetLastError();
        const dim3 grid((links + kLinkThreads / 2 - 1) / (kLinkThreads / 2));  // two lanes a link
        if (err == hipSuccess) {
            const bool trace = d_flits != nullptr;
            if (small) {
                if (trace) {
                    hipLaunchKernelGGL((k_link<kSmallMsg, kSmallFlit, true>), grid,
                                       dim3(kLinkThreads), 0, stream, a);
                } else {
                    hipLaunchKernelGGL((k_link<kSmallMsg, kSmallFlit>), grid, dim3(kLinkThreads),
                                       0, stream, a);
                }
            } else if (lds) {
                if (trace) {
                    hipLaunchKernelGGL((k_link<kLargeMsg, kLargeFlit, true>), grid,
                                       dim3(kLinkThreads), 0, stream, a);
                } else {
                    hipLaunchKernelGGL((k_link<kLargeMsg, kLargeFlit>), grid, dim3(kLinkThreads),
                                       0, stream, a);
                }
            } else if (trace) {
                hipLaunchKernelGGL((k_link<0, 0, true>), grid, dim3(kLinkThreads), 0, stream, a);
            } else {
                hipLaunchKernelGGL((k_link<0, 0>), grid, dim3(kLinkThreads), 0, stream, a);
            }
            err = hipGetLastError();
        }
        if (err == hipSuccess) {
            err = hipMemcpyAsync(&h_err, a.error, 4, hipMemcpyDeviceToHost, stream);
        }
    }
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) {
        return HBFSIM_CUDA_ERROR;
    }
    return h_err == 0 ? HBFSIM_OK : HBFSIM_INVALID_ARGUMENT;
}

}  // namespace hbfamd
