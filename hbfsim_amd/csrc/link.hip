// link.hip -- the UCIe Streaming / AoU link (src/ucie/link.cpp:1-203) for
// batches of independent links on gfx950 (MI355X).
//
// One thread runs one link's event loop: AR requests (3 AoU granules) and R
// returns (14) queue per direction; a direction sends a Format 6 flit of 48
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
    std::uint64_t* counters;       // [links][2][8]
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
// (the fast form: at most kLdsMsgSlots messages admitted per direction and
// kLdsFlitSlots flits in flight, which the reference defaults and every
// propagation delay up to 5 flit times meet) or in HBM: the message times
// in place of their ready times in the split lists, the flit rings in a
// scratch buffer.
constexpr std::uint32_t kLdsMsgSlots = 16;
constexpr std::uint32_t kLdsFlitSlots = 8;

template <bool kLds>
__global__ __launch_bounds__(kLinkThreads) void k_link(LinkArgs a)
{
    __shared__ std::uint64_t s_msg_t[kLds ? 2 * kLdsMsgSlots * kLinkThreads : 1];
    __shared__ std::uint32_t s_msg_i[kLds ? 2 * kLdsMsgSlots * kLinkThreads : 1];
    __shared__ std::uint64_t s_fl_t[kLds ? 2 * kLdsFlitSlots * kLinkThreads : 1];
    __shared__ std::uint32_t s_fl_i[kLds ? 2 * kLdsFlitSlots * kLinkThreads : 1];
    const std::uint32_t lane = threadIdx.x;
    const std::uint32_t l = blockIdx.x * kLinkThreads + lane;
    if (l >= a.links) {
        return;
    }
    const std::uint64_t ar = a.n_ar[l];
    if (ar == kBadLink) {
        return;  // refused by the split pass
    }
    const std::uint64_t b = a.first[l], e = a.first[l + 1];
    const std::uint64_t base[2] = {b, b + ar};     // each direction's list
    // the split pass refuses links of 2^32 messages or more
    const std::uint32_t count[2] = {static_cast<std::uint32_t>(ar),
                                    static_cast<std::uint32_t>(e - b - ar)};
    const std::uint32_t size[2] = {3u, 14u};
    const std::uint32_t M = a.max_accepted;
    // flit slot s of direction d: LDS lane-minor (conflict-free), HBM link-major
    auto fl_t = [&](std::uint32_t d, std::uint32_t s) -> std::uint64_t& {
        if constexpr (kLds) {
            return s_fl_t[(d * kLdsFlitSlots + s) * kLinkThreads + lane];
        } else {
            return a.ring_time[(2ull * l + d) * a.ring + s];
        }
    };
    auto fl_i = [&](std::uint32_t d, std::uint32_t s) -> std::uint32_t& {
        if constexpr (kLds) {
            return s_fl_i[(d * kLdsFlitSlots + s) * kLinkThreads + lane];
        } else {
            return a.ring_info[(2ull * l + d) * a.ring + s];
        }
    };
    // message k of direction d (LDS slot s = k mod max_accepted)
    auto msg_t = [&](std::uint32_t d, std::uint32_t k, std::uint32_t s) -> std::uint64_t& {
        if constexpr (kLds) {
            return s_msg_t[(d * kLdsMsgSlots + s) * kLinkThreads + lane];
        } else {
            return a.part_time[base[d] + k];
        }
    };
    auto msg_i = [&](std::uint32_t d, std::uint32_t k, std::uint32_t s) -> std::uint32_t {
        if constexpr (kLds) {
            return s_msg_i[(d * kLdsMsgSlots + s) * kLinkThreads + lane];
        } else {
            return a.part_index[base[d] + k];
        }
    };
    auto wrap = [&](std::uint32_t s) -> std::uint32_t { return s + 1 == M ? 0u : s + 1; };
    // per direction: messages admitted, arrived, sent, delivered, consumed,
    // with their LDS slots; the next admission's ready time and index
    std::uint32_t n_adm[2] = {0, 0}, n_arr[2] = {0, 0}, n_done[2] = {0, 0};
    std::uint32_t n_dlv[2] = {0, 0}, n_con[2] = {0, 0};
    std::uint32_t s_adm[2] = {0, 0}, s_arr[2] = {0, 0}, s_dlv[2] = {0, 0}, s_con[2] = {0, 0};
    std::uint64_t next_ready[2] = {0, 0};
    std::uint32_t next_index[2] = {0, 0};
    std::uint64_t last_ready[2] = {0, 0};
    std::uint32_t h_rem[2], h_started[2] = {0, 0};
    std::uint64_t cursor[2] = {0, 0};
    std::uint32_t credits[2] = {a.credit0[0], a.credit0[1]};
    std::uint32_t gp[2] = {0, 0};  // credits to grant back on direction d's flits
    std::uint32_t rh[2] = {0, 0}, rn[2] = {0, 0};  // flit ring head, entries
    std::uint64_t flits[2] = {0, 0}, gran[2] = {0, 0}, credit_only[2] = {0, 0};
    for (std::uint32_t d = 0; d < 2; ++d) {
        h_rem[d] = size[d];
        if (count[d] != 0) {
            next_ready[d] = a.part_time[base[d]];
            next_index[d] = kLds ? a.part_index[base[d]] : 0u;
        }
    }
    std::uint64_t now = 0;
    std::uint32_t err = 0;
    const std::uint64_t cap = 64ull * (e - b) + 4096;
    for (std::uint64_t it = 0; err == 0; ++it) {
        if (it >= cap) {
            err = 2;
            break;
        }
        // the caller admits waiting messages while a direction has room
        for (std::uint32_t d = 0; d < 2; ++d) {
            while (n_adm[d] < count[d] && n_adm[d] - n_con[d] < M) {
                const std::uint64_t r = next_ready[d];
                if (r < last_ready[d]) {
                    err = 1;  // a direction's ready times must not decrease
                }
                last_ready[d] = r;
                msg_t(d, n_adm[d], s_adm[d]) = r > now ? r : now;
                if constexpr (kLds) {
                    s_msg_i[(d * kLdsMsgSlots + s_adm[d]) * kLinkThreads + lane] = next_index[d];
                    s_adm[d] = wrap(s_adm[d]);
                }
                ++n_adm[d];
                if (n_adm[d] < count[d]) {  // fetch the next admission ahead of its use
                    next_ready[d] = a.part_time[base[d] + n_adm[d]];
                    if constexpr (kLds) {
                        next_index[d] = a.part_index[base[d] + n_adm[d]];
                    }
                }
            }
        }
        if (err != 0) {
            break;
        }
        // the next event
        bool any = false;
        std::uint64_t t = ~0ull;
        for (std::uint32_t d = 0; d < 2; ++d) {
            if (n_arr[d] < n_adm[d]) {
                const std::uint64_t x = msg_t(d, n_arr[d], s_arr[d]);
                t = x < t ? x : t;
                any = true;
            }
            if (rn[d] != 0) {
                const std::uint64_t x = fl_t(d, rh[d]);
                t = x < t ? x : t;
                any = true;
            }
            if (n_con[d] < n_dlv[d]) {
                const std::uint64_t dv = msg_t(d, n_con[d], s_con[d]);
                if (dv > ~0ull - a.delay[d]) {
                    err = 1;
                }
                const std::uint64_t x = dv + a.delay[d];
                t = x < t ? x : t;
                any = true;
            }
            if (cursor[d] > now && (n_arr[d] > n_done[d] || gp[d] != 0)) {
                t = cursor[d] < t ? cursor[d] : t;
                any = true;
            }
        }
        if (err != 0 || !any) {
            break;
        }
        now = t;
        // every arrival, delivery and consume scheduled at `now`; consumes
        // of messages this step delivers wait for the next step
        const std::uint32_t dlv_before[2] = {n_dlv[0], n_dlv[1]};
        for (std::uint32_t d = 0; d < 2; ++d) {
            while (n_arr[d] < n_adm[d] && msg_t(d, n_arr[d], s_arr[d]) == now) {
                ++n_arr[d];
                s_arr[d] = wrap(s_arr[d]);
            }
        }
        for (std::uint32_t d = 0; d < 2; ++d) {
            if (rn[d] != 0 && fl_t(d, rh[d]) == now) {
                const std::uint32_t info = fl_i(d, rh[d]);
                const std::uint32_t grant = info >> 16, done = info & 0xffffu;
                const std::uint32_t o = d ^ 1u;  // the grant is for the other direction
                if (grant > a.credit0[o] - credits[o]) {
                    err = 1;
                }
                credits[o] += grant;
                for (std::uint32_t k = 0; k < done; ++k) {
                    msg_t(d, n_dlv[d], s_dlv[d]) = now;
                    a.delivered[b + msg_i(d, n_dlv[d], s_dlv[d])] = now;
                    ++n_dlv[d];
                    s_dlv[d] = wrap(s_dlv[d]);
                }
                rh[d] = rh[d] + 1 == a.ring ? 0u : rh[d] + 1;
                --rn[d];
            }
        }
        for (std::uint32_t d = 0; d < 2; ++d) {
            while (n_con[d] < dlv_before[d] && msg_t(d, n_con[d], s_con[d]) + a.delay[d] == now) {
                const std::uint32_t o = d ^ 1u;
                if (gp[o] > 65535u - size[d]) {
                    err = 1;
                    break;
                }
                gp[o] += size[d];
                ++n_con[d];
                s_con[d] = wrap(s_con[d]);
            }
        }
        if (err != 0) {
            break;
        }
        // both directions send (link.cpp send_ready)
        for (std::uint32_t d = 0; d < 2; ++d) {
            if (cursor[d] > now) {
                continue;
            }
            std::uint32_t used = 0, done = 0;
            while (n_arr[d] > n_done[d] && used < 48) {
                if (!h_started[d]) {
                    if (credits[d] < size[d]) {
                        break;
                    }
                    credits[d] -= size[d];
                    h_started[d] = 1;
                }
                const std::uint32_t frag = 48 - used < h_rem[d] ? 48 - used : h_rem[d];
                used += frag;
                h_rem[d] -= frag;
                if (h_rem[d] == 0) {
                    ++done;
                    ++n_done[d];
                    h_rem[d] = size[d];
                    h_started[d] = 0;
                }
            }
            const std::uint32_t grant = legal_grant(gp[d]);
            if (used == 0 && grant == 0) {
                continue;
            }
            gp[d] -= grant;
            if (now > ~0ull - a.ser || now + a.ser > ~0ull - a.prop || rn[d] == a.ring) {
                err = 1;
                break;
            }
            cursor[d] = now + a.ser;
            const std::uint32_t slot = rh[d] + rn[d] < a.ring ? rh[d] + rn[d]
                                                               : rh[d] + rn[d] - a.ring;
            fl_t(d, slot) = cursor[d] + a.prop;
            fl_i(d, slot) = (grant << 16) | done;
            ++rn[d];
            ++flits[d];
            gran[d] += used;
            credit_only[d] += used == 0 ? 1u : 0u;
        }
    }
    if (err != 0) {
        atomicMax(a.error, err);
    }
    for (std::uint32_t d = 0; d < 2; ++d) {
        std::uint64_t* c = a.counters + (2ull * l + d) * 8;
        c[0] = flits[d];
        c[1] = 256 * flits[d];
        c[2] = 2 * flits[d];
        c[3] = 4 * flits[d];
        c[4] = 10 * flits[d];
        c[5] = 5 * gran[d];
        c[6] = 5 * (48 * flits[d] - gran[d]);
        c[7] = credit_only[d];
    }
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
             std::uint64_t* d_delivered, hbfsim_amd_link_counters* d_counters, void* stream_ptr)
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
    const bool lds = p.max_accepted <= kLdsMsgSlots && ring <= kLdsFlitSlots;
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
        a.part_time = reinterpret_cast<std::uint64_t*>(scratch + o_time);
        a.part_index = reinterpret_cast<std::uint32_t*>(scratch + o_index);
        a.n_ar = reinterpret_cast<std::uint64_t*>(scratch + o_ar);
        a.ring_time = lds ? nullptr : reinterpret_cast<std::uint64_t*>(scratch + o_rt);
        a.ring_info = lds ? nullptr : reinterpret_cast<std::uint32_t*>(scratch + o_ri);
        a.error = reinterpret_cast<std::uint32_t*>(scratch + o_err);
        hipLaunchKernelGGL(k_link_split, dim3((links + kSplitWaves - 1) / kSplitWaves),
                           dim3(kSplitWaves * 64), 0, stream, a);
        err = hipGetLastError();
        const dim3 grid((links + kLinkThreads - 1) / kLinkThreads);
        if (err == hipSuccess) {
            if (lds) {
                hipLaunchKernelGGL(k_link<true>, grid, dim3(kLinkThreads), 0, stream, a);
            } else {
                hipLaunchKernelGGL(k_link<false>, grid, dim3(kLinkThreads), 0, stream, a);
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
