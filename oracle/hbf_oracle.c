/*
 * hbf_oracle.c -- CPU restatement of HBFSim's per-access timing path.
 *
 * TEST INFRASTRUCTURE ONLY (see hbf_oracle.h).  Plain C11, no GPU, no
 * dependency on the product library.  Written from the behaviour of the
 * cited reference functions; nothing here is shipped or used as a fallback.
 */
#include "hbf_oracle.h"

#include <omp.h>

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* hbf_device.cuh:729-736.  SplitMix64 finaliser (public constants). */
uint64_t orc_fast_hash(uint64_t value)
{
    value += 0x9e3779b97f4a7c15ULL;
    value = (value ^ (value >> 30)) * 0xbf58476d1ce4e5b9ULL;
    value = (value ^ (value >> 27)) * 0x94d049bb133111ebULL;
    return value ^ (value >> 31);
}

/* hbf_device.cuh:738-744 */
int orc_hybrid_reference_sample(uint64_t sequence, uint32_t warmup,
                                uint64_t threshold, uint64_t key)
{
    return sequence < warmup ||
           (threshold != 0 && orc_fast_hash(sequence ^ key) <= threshold);
}

/* context.cpp:975-981: rate * UINT64_MAX in long double, saturating at 1. */
uint64_t orc_sample_threshold(double rate)
{
    if (rate >= 1.0) {
        return UINT64_MAX;
    }
    return (uint64_t)((long double)rate * (long double)UINT64_MAX);
}

/* hbf_device.cuh:746-756: ceil(bytes * 1e9 / bandwidth) ns, 0 if either is 0 */
uint64_t orc_fast_transfer_ns(uint32_t bytes, uint64_t bandwidth)
{
    if (bytes == 0 || bandwidth == 0) {
        return 0;
    }
    const uint64_t numerator = (uint64_t)bytes * 1000000000ULL;
    return (numerator + bandwidth - 1) / bandwidth;
}

/* hbf_device.cuh:797-816: the later of latency and transfer, not the sum */
uint64_t orc_fast_service_ns(uint64_t base_ns, uint32_t bytes,
                             uint64_t bandwidth)
{
    const uint64_t transfer = orc_fast_transfer_ns(bytes, bandwidth);
    return transfer > base_ns ? transfer : base_ns;
}

/* hbf_device.cuh:946-957 */
uint64_t orc_saturating_add(uint64_t a, uint64_t b)
{
    return b > UINT64_MAX - a ? UINT64_MAX : a + b;
}

uint64_t orc_saturating_multiply(uint64_t a, uint32_t b)
{
    return b != 0 && a > UINT64_MAX / b ? UINT64_MAX : a * b;
}

/* hbf_device.cuh:826-841: upper_bound(base) - 1, or count when none */
uint32_t orc_find_range_index(const orc_range* ranges, uint32_t count,
                              uint64_t address)
{
    uint32_t lo = 0, hi = count;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (ranges[mid].base <= address) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo == 0 ? count : lo - 1;
}

/* hbf_device.cuh:843-860 */
int orc_access_supported(const orc_range* r, uint64_t address, uint32_t bytes,
                         uint32_t operation)
{
    if (bytes == 0 || operation > 1 || (r->mode != 1 && r->mode != 2) ||
        r->page_bytes == 0 || r->page_bytes > UINT32_MAX ||
        r->length > UINT64_MAX - r->base || address < r->base ||
        address - r->base >= r->length || bytes > UINT64_MAX - address ||
        address + bytes > r->base + r->length ||
        (r->permissions & (1u << operation)) == 0) {
        return 0;
    }
    const uint64_t offset = address - r->base;
    const uint64_t last = offset + bytes - 1;
    return offset / r->page_bytes == last / r->page_bytes;
}

/* hbf_device.cuh:873-884 */
int orc_range_overlaps(const orc_range* r, uint64_t address, uint32_t bytes)
{
    if (bytes == 0 || r->length == 0 || r->base > UINT64_MAX - r->length ||
        address > UINT64_MAX - bytes) {
        return 0;
    }
    return address < r->base + r->length && r->base < address + bytes;
}

/* hbf_device.cuh:895-909 */
int orc_span_touches_any_range(const orc_range* ranges, uint32_t count,
                               uint64_t address, uint32_t bytes)
{
    if (ranges == NULL || count == 0 || bytes == 0) {
        return 0;
    }
    const uint32_t index = orc_find_range_index(ranges, count, address);
    if (index != count && orc_range_overlaps(&ranges[index], address, bytes)) {
        return 1;
    }
    const uint32_t successor = index == count ? 0u : index + 1u;
    return successor < count &&
           orc_range_overlaps(&ranges[successor], address, bytes);
}

/* hbf_device.cuh:929-944 */
orc_media orc_media_descriptor(const orc_range* r, uint64_t address,
                               uint32_t bytes, uint32_t operation)
{
    orc_media m = {0, 0, 0};
    if (!orc_access_supported(r, address, bytes, operation)) {
        return m;
    }
    const uint64_t page_offset =
        ((address - r->base) / r->page_bytes) * r->page_bytes;
    if (page_offset > UINT64_MAX - r->file_offset) {
        return m;
    }
    m.logical_address = r->file_offset + page_offset;
    m.bytes = (uint32_t)r->page_bytes;
    m.valid = 1;
    return m;
}

/* The resolver's classification order, hbf_device.cu:1081-1165:
 *   1. start-address lookup; if the start lies outside every range, the
 *      access is rejected when its span reaches into the successor range
 *      (:1094-1108), else it bypasses at native speed (:1128-1136);
 *   2. inside a range, media_descriptor must be valid (:1151-1165).
 * Record bytes wider than 32 bits cannot be described by the device ABI
 * (u32 bytes) and are rejected. */
uint32_t orc_classify(const orc_range* ranges, uint32_t count,
                      uint64_t address, uint64_t bytes, uint32_t operation,
                      uint32_t* range_index)
{
    const uint32_t b32 = bytes > UINT32_MAX ? 0u : (uint32_t)bytes;
    const uint32_t index = orc_find_range_index(ranges, count, address);
    if (index == count || address < ranges[index].base ||
        address - ranges[index].base >= ranges[index].length) {
        const uint32_t successor = index == count ? 0u : index + 1u;
        if (bytes > UINT32_MAX ||
            (successor < count &&
             orc_range_overlaps(&ranges[successor], address, b32))) {
            return ORC_UNSUPPORTED;
        }
        return ORC_BYPASS;
    }
    if (bytes > UINT32_MAX) {
        return ORC_UNSUPPORTED;
    }
    const orc_media m = orc_media_descriptor(&ranges[index], address, b32,
                                             operation);
    if (!m.valid) {
        return ORC_UNSUPPORTED;
    }
    *range_index = index;
    return ORC_MODELED;
}

/* hbf_device.cuh:959-978 */
uint64_t orc_ceiling_scaled_delta(uint64_t delta, uint32_t offset,
                                  uint32_t span)
{
    if (delta == 0 || offset == 0) {
        return 0;
    }
    if (span == 0) {
        return UINT64_MAX;
    }
    const uint64_t quotient = delta / span;
    const uint64_t remainder = delta % span;
    const uint64_t integral = orc_saturating_multiply(quotient, offset);
    const uint64_t fractional =
        (remainder * (uint64_t)offset + span - 1) / span;
    return orc_saturating_add(integral, fractional);
}

/* hbf_device.cuh:980-1016: piecewise-linear cumulative curve with ceiling
 * interpolation; beyond the last point extrapolates the last segment. */
uint64_t orc_empirical_cumulative_ns(const uint32_t* pages,
                                     const uint64_t* cumulative,
                                     uint32_t count, uint32_t run_pages)
{
    if (run_pages == 0) {
        return 0;
    }
    if (pages == NULL || cumulative == NULL || count == 0) {
        return UINT64_MAX;
    }
    uint32_t right = 0;
    while (right < count && run_pages > pages[right]) {
        ++right;
    }
    if (right == count) {
        right = count - 1;
    }
    uint32_t left_pages = 0;
    uint64_t left_ns = 0;
    if (right != 0) {
        left_pages = pages[right - 1];
        left_ns = cumulative[right - 1];
    }
    if (run_pages > pages[right] && count > 1) {
        left_pages = pages[count - 2];
        left_ns = cumulative[count - 2];
        right = count - 1;
    }
    if (pages[right] <= left_pages || cumulative[right] < left_ns ||
        run_pages < left_pages) {
        return UINT64_MAX;
    }
    const uint64_t inc = orc_ceiling_scaled_delta(
        cumulative[right] - left_ns, run_pages - left_pages,
        pages[right] - left_pages);
    return orc_saturating_add(left_ns, inc);
}

/* hbf_device.cuh:1018-1029 */
uint64_t orc_empirical_service_ns(const uint32_t* pages,
                                  const uint64_t* cumulative, uint32_t count,
                                  uint32_t run_pages)
{
    if (run_pages == 0) {
        return 0;
    }
    const uint64_t cur =
        orc_empirical_cumulative_ns(pages, cumulative, count, run_pages);
    const uint64_t prev =
        orc_empirical_cumulative_ns(pages, cumulative, count, run_pages - 1);
    return cur < prev ? UINT64_MAX : cur - prev;
}

#define ORC_BURST_RUN_MASK 1023ULL
#define ORC_MAX_EMPIRICAL_PAGE ((1ULL << 53) - 2)

/* hbf_device.cuh:1031-1080: packed = (page+1) << 11 | op << 10 | run */
int orc_update_empirical_burst(uint64_t previous, uint64_t page,
                               uint32_t operation, uint64_t* packed,
                               uint32_t* run_pages)
{
    if (page > ORC_MAX_EMPIRICAL_PAGE || operation > 1) {
        *packed = previous;
        *run_pages = 0;
        return 0;
    }
    uint32_t run = 1;
    const uint64_t prev_plus_one = previous >> 11;
    const uint64_t prev_page = prev_plus_one == 0 ? UINT64_MAX
                                                  : prev_plus_one - 1;
    const uint32_t prev_run = (uint32_t)(previous & ORC_BURST_RUN_MASK);
    const uint32_t prev_op = (uint32_t)((previous >> 10) & 1u);
    if (previous != 0 && prev_run != 0 && prev_op == operation &&
        prev_page != UINT64_MAX && prev_page + 1 == page) {
        run = prev_run == ORC_BURST_RUN_MASK ? prev_run : prev_run + 1;
    }
    *packed = ((page + 1) << 11) | ((uint64_t)operation << 10) | run;
    *run_pages = run;
    return 1;
}

/* hbf_device.cuh:1089-1111 */
int orc_empirical_control_valid(const orc_empirical* e)
{
    if (e->flags != 1 || e->point_count != 6 || e->program_latency_ns == 0) {
        return 0;
    }
    for (uint32_t i = 0; i < 6; ++i) {
        if (e->pages[i] == 0 || e->cumulative_ns[i] == 0 ||
            (i != 0 && e->pages[i] <= e->pages[i - 1]) ||
            (i != 0 && e->cumulative_ns[i] <= e->cumulative_ns[i - 1])) {
            return 0;
        }
    }
    return e->pages[5] <= ORC_BURST_RUN_MASK;
}

/* hbf_device.cuh:1113-1140 */
int orc_empirical_request_service(const orc_empirical* e, uint64_t previous,
                                  uint64_t page, uint32_t operation,
                                  uint64_t* service_ns, uint64_t* packed,
                                  uint32_t* run_pages)
{
    if (!orc_empirical_control_valid(e)) {
        return 0;
    }
    if (!orc_update_empirical_burst(previous, page, operation, packed,
                                    run_pages)) {
        return 0;
    }
    *service_ns = operation == 0
                      ? orc_empirical_service_ns(e->pages, e->cumulative_ns,
                                                 e->point_count, *run_pages)
                      : e->program_latency_ns;
    return 1;
}

/* ---- range registry: range_table.cpp:17-198 ------------------------- */
orc_range_table* orc_range_table_create(uint64_t page_bytes,
                                        uint64_t media_capacity)
{
    orc_range_table* t = (orc_range_table*)calloc(1, sizeof(*t));
    if (t == NULL) {
        return NULL;
    }
    t->records = (orc_range*)calloc(ORC_RANGE_CAPACITY, sizeof(orc_range));
    if (t->records == NULL) {
        free(t);
        return NULL;
    }
    t->next_range_id = 1;
    t->page_bytes = page_bytes;
    t->media_capacity = media_capacity;
    return t;
}

void orc_range_table_destroy(orc_range_table* t)
{
    if (t != NULL) {
        free(t->records);
        free(t);
    }
}

/* range_table.cpp:17-118: validation, media extent, overlap, publish */
int orc_range_table_add(orc_range_table* t, uint64_t base, uint64_t length,
                        uint32_t mode, uint32_t permissions,
                        uint32_t cache_policy, uint32_t stream_id)
{
    if (base == 0 || length == 0 || t->page_bytes == 0 ||
        length > UINT64_MAX - base || permissions == 0 ||
        (permissions & ~3u) != 0 || cache_policy != 0) {
        return 1;
    }
    if (mode != 1 && mode != 2) {
        return 1;
    }
    if (t->count == ORC_RANGE_CAPACITY) {
        return 5;
    }
    if (length > UINT64_MAX - (t->page_bytes - 1)) {
        return 5;
    }
    const uint64_t extent =
        ((length + t->page_bytes - 1) / t->page_bytes) * t->page_bytes;
    if (t->next_file_offset > t->media_capacity ||
        extent > t->media_capacity - t->next_file_offset) {
        return 5;
    }
    /* lower_bound on base */
    uint32_t lo = 0, hi = t->count;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (t->records[mid].base < base) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    const uint32_t index = lo;
    const uint64_t end = base + length;
    if ((index != 0 && t->records[index - 1].base +
                               t->records[index - 1].length > base) ||
        (index != t->count && end > t->records[index].base)) {
        return 1;
    }
    memmove(&t->records[index + 1], &t->records[index],
            (size_t)(t->count - index) * sizeof(orc_range));
    orc_range r;
    memset(&r, 0, sizeof(r));
    r.base = base;
    r.length = length;
    r.file_offset = t->next_file_offset;
    r.range_id = t->next_range_id;
    r.mode = mode;
    r.permissions = permissions;
    r.cache_policy = cache_policy;
    r.stream_id = stream_id;
    r.page_bytes = t->page_bytes;
    t->records[index] = r;
    t->count += 1;
    t->next_range_id += 1;
    t->next_file_offset += extent;
    return 0;
}

/* range_table.cpp:120-171 */
int orc_range_table_remove(orc_range_table* t, uint64_t base)
{
    if (base == 0) {
        return 1;
    }
    uint32_t lo = 0, hi = t->count;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (t->records[mid].base < base) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    if (lo == t->count || t->records[lo].base != base) {
        return 1;
    }
    memmove(&t->records[lo], &t->records[lo + 1],
            (size_t)(t->count - lo - 1) * sizeof(orc_range));
    t->count -= 1;
    memset(&t->records[t->count], 0, sizeof(orc_range));
    return 0;
}

/* range_table.cpp:173-198 */
int orc_range_table_lookup(const orc_range_table* t, uint64_t address,
                           uint32_t bytes, uint32_t* index)
{
    if (bytes == 0 || t->count == 0) {
        return 0;
    }
    uint32_t lo = 0, hi = t->count; /* upper_bound */
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (address < t->records[mid].base) {
            hi = mid;
        } else {
            lo = mid + 1;
        }
    }
    if (lo == 0) {
        return 0;
    }
    const orc_range* r = &t->records[lo - 1];
    if (address < r->base || address - r->base >= r->length) {
        return 0;
    }
    *index = lo - 1;
    if (bytes > UINT64_MAX - address || address + bytes > r->base + r->length) {
        return 2;
    }
    return 1;
}

/* ---- striping ------------------------------------------------------- */
/* MQSim's plane allocation scheme names the axis that advances fastest
 * first (profile.hpp:51-77; the CWDP case is spelled out by
 * bank_layout.cpp:59-72 as channel = lpa % C, chip = (lpa / C) % chips). */
uint64_t orc_stripe(uint64_t page, const uint32_t order[4],
                    const uint32_t sizes[4], uint32_t coords[4])
{
    uint64_t rem = page;
    for (int i = 0; i < 4; ++i) {
        const uint32_t axis = order[i];
        coords[axis] = (uint32_t)(rem % sizes[axis]);
        rem /= sizes[axis];
    }
    return rem; /* row (page index within the plane) */
}

int orc_parse_scheme(const char* name, uint32_t order[4])
{
    if (name == NULL || strlen(name) != 4) {
        return 0;
    }
    uint32_t seen = 0;
    for (int i = 0; i < 4; ++i) {
        uint32_t axis;
        switch (name[i]) {
        case 'C': axis = 0; break;
        case 'W': axis = 1; break;
        case 'D': axis = 2; break;
        case 'P': axis = 3; break;
        default: return 0;
        }
        if (seen & (1u << axis)) {
            return 0;
        }
        seen |= 1u << axis;
        order[i] = axis;
    }
    return 1;
}

/* bank_layout.cpp:48-57 */
uint64_t orc_hbf_media_lpa(uint64_t q, uint32_t module, uint32_t channels)
{
    return q * channels + module;
}

/* bank_layout.cpp:59-72 */
void orc_hbf_cold_read_bank(uint64_t lpa, uint32_t channels,
                            uint32_t core_dies, uint32_t banks,
                            uint32_t* channel, uint32_t* core_die,
                            uint32_t* bank, uint32_t* chip)
{
    *channel = (uint32_t)(lpa % channels);
    const uint32_t c = (uint32_t)((lpa / channels) % (core_dies * banks));
    *chip = c;
    *core_die = c / banks;
    *bank = c % banks;
}

/* ---- multi-resource engine ----------------------------------------- */
static uint64_t xfer_ps(const orc_engine_params* p, uint64_t bytes)
{
    /* q * ceil(bytes * num / den): bytes at the per-channel bandwidth,
     * rounded up to whole quanta (q = 1000 reproduces the reference's
     * whole-nanosecond transfer times, hbf_device.cuh:746-756). */
    const u128 prod = (u128)bytes * p->xfer_num;
    return p->xfer_quantum *
           (uint64_t)((prod + p->xfer_den - 1) / p->xfer_den);
}

static uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

/* Page-buffer slot rule per plane.  slots==1: one page register.
 * slots==2: device_coalescer.cpp:134-168 -- a miss takes the first empty
 * slot, else the lowest-index unpinned slot (slot 0).  Nothing is pinned
 * here because a plane finishes one sense before the next begins. */
static int pagebuf_access(uint64_t* tags, uint32_t slots, uint64_t page)
{
    const uint64_t tag = page + 1;
    for (uint32_t k = 0; k < slots; ++k) {
        if (tags[k] == tag) {
            return 1;
        }
    }
    for (uint32_t k = 0; k < slots; ++k) {
        if (tags[k] == 0) {
            tags[k] = tag;
            return 0;
        }
    }
    if (slots > 0) {
        tags[0] = tag;
    }
    return 0;
}

void orc_pagebuf_sequence(const uint64_t* pages, size_t n, uint32_t slots,
                          uint8_t* hits)
{
    uint64_t tags[2] = {0, 0};
    for (size_t i = 0; i < n; ++i) {
        hits[i] = (uint8_t)pagebuf_access(tags, slots, pages[i]);
    }
}

static void add128(orc_engine_report* r, uint64_t v)
{
    const uint64_t lo = r->latency_sum_lo + v;
    r->latency_sum_hi += lo < r->latency_sum_lo;
    r->latency_sum_lo = lo;
}

/* Per-record decode shared by the sequential and parallel oracles. */
typedef struct decoded {
    uint32_t cls;
    uint32_t op;
    uint32_t plane;   /* global plane id */
    uint32_t channel;
    uint64_t page;    /* media page number */
    uint64_t issue;
    uint64_t xfer;
    uint64_t svc_miss;  /* plane service when the page is not buffered */
    uint64_t svc_hit;   /* plane service when it is */
    uint32_t range_id;
} decoded;

static void decode(const orc_engine_params* p, const orc_range* ranges,
                   uint32_t count, const orc_record* rec, uint64_t base_ps,
                   decoded* d)
{
    memset(d, 0, sizeof(*d));
    const uint32_t op = (uint32_t)(rec->flags & 0xffu);
    uint32_t index = 0;
    d->issue = base_ps + rec->issue_ps;
    d->op = op;
    if (p->media_records && op == ORC_OP_REFRESH && (rec->flags & ORC_FLAG_MEDIA) != 0) {
        /* refresh of media page `addr`: read it out and program it back
         * (cpu_service.cpp:181-212's read -> program pair as one job) */
        const uint64_t page = rec->addr;
        if (rec->bytes == 0 || rec->bytes > 0xffffffffULL ||
            (p->media_pages != 0 && page >= p->media_pages) ||
            page >= (UINT64_MAX >> p->page_shift)) {
            d->cls = ORC_UNSUPPORTED;
            return;
        }
        d->cls = ORC_MODELED;
        d->page = page;
        const uint32_t sz[4] = {p->channels, p->ways, p->dies, p->planes};
        uint32_t cc[4];
        orc_stripe(page, p->order, sz, cc);
        d->channel = cc[0];
        d->plane = ((cc[0] * p->ways + cc[1]) * p->dies + cc[2]) * p->planes + cc[3];
        d->xfer = xfer_ps(p, rec->bytes);
        d->svc_miss = d->svc_hit = p->read_ps + p->program_ps;
        return;
    }
    d->cls = orc_classify(ranges, count, rec->addr, rec->bytes, op, &index);
    if (d->cls != ORC_MODELED) {
        return;
    }
    const orc_range* r = &ranges[index];
    const uint64_t media = r->file_offset + (rec->addr - r->base);
    const uint64_t page_bytes = 1ULL << p->page_shift;
    d->page = media >> p->page_shift;
    d->range_id = r->range_id;
    const uint32_t sizes[4] = {p->channels, p->ways, p->dies, p->planes};
    uint32_t c[4];
    orc_stripe(d->page, p->order, sizes, c);
    d->channel = c[0];
    d->plane = ((c[0] * p->ways + c[1]) * p->dies + c[2]) * p->planes + c[3];
    const uint64_t xbytes = p->transfer_page ? page_bytes : rec->bytes;
    d->xfer = xfer_ps(p, xbytes);
    if (op == 0) {
        d->svc_miss = p->read_ps;
        d->svc_hit = 0;
    } else {
        const uint64_t off = media & (page_bytes - 1);
        const int fill = off + rec->bytes == page_bytes;
        d->svc_miss = d->svc_hit =
            (fill || p->program_every_write) ? p->program_ps : 0;
    }
}

static int engine_params_ok(const orc_engine_params* p)
{
    return p->channels && p->ways && p->dies && p->planes &&
           p->page_shift >= 9 && p->page_shift < 63 && p->page_buffers <= 2 &&
           p->xfer_den != 0 && p->xfer_quantum != 0;
}

static uint32_t group_of(const orc_engine_params* p, const orc_record* r)
{
    return p->warp_grouping ? (uint32_t)(r->flags >> 32) : 0u;
}

/* A group is a maximal run of consecutive records with one nonzero id: at
 * most ORC_GROUP_MAX records, all with one issue time. */
static int groups_valid(const orc_engine_params* p, const orc_record* records, size_t n)
{
    size_t len = 0;
    for (size_t i = 0; i < n; ++i) {
        const uint32_t g = group_of(p, &records[i]);
        if (g != 0 && i > 0 && len != 0 && g == group_of(p, &records[i - 1])) {
            if (len == ORC_GROUP_MAX || records[i].issue_ps != records[i - 1].issue_ps) {
                return 0;
            }
            ++len;
        } else {
            len = g != 0;
        }
    }
    return 1;
}

/* The engine over a stream whose records are served in stream position
 * order (orc_engine_run sorts any other stream first). */
static int engine_run_in_order(const orc_engine_params* p, const orc_range* ranges,
                               uint32_t range_count, const orc_record* records, size_t n,
                               uint64_t base_ps, orc_engine_state* s, uint64_t* completion,
                               uint8_t* status, orc_engine_report* rep)
{
    if (!engine_params_ok(p)) {
        return 1;
    }
    if (p->model == ORC_MODEL_FAST_EMPIRICAL &&
        (!orc_empirical_control_valid(&p->empirical) || p->page_shift != 12)) {
        return 5;
    }
    if (p->warp_grouping && !groups_valid(p, records, n)) {
        return 6;
    }
    const uint32_t slots = p->page_buffers;
    /* the current group's requests: (range, page) and the record that made it */
    size_t g_lead[ORC_GROUP_MAX];
    uint64_t g_page[ORC_GROUP_MAX];
    uint32_t g_range[ORC_GROUP_MAX];
    uint32_t g_n = 0;
    for (size_t i = 0; i < n; ++i) {
        decoded d;
        decode(p, ranges, range_count, &records[i], base_ps, &d);
        rep->records += 1;
        uint8_t st = (uint8_t)d.cls;
        const uint32_t g = group_of(p, &records[i]);
        if (g == 0 || i == 0 || g != group_of(p, &records[i - 1])) {
            g_n = 0;  /* a new group (or none) */
        }
        if (g != 0 && d.cls == ORC_MODELED) {
            uint32_t k = 0;
            while (k < g_n && !(g_range[k] == d.range_id && g_page[k] == d.page)) {
                ++k;
            }
            if (k < g_n) {
                /* a lane of the request of record g_lead[k] */
                const uint64_t done = completion[g_lead[k]];
                completion[i] = done;
                rep->modeled += 1;
                rep->grouped += 1;
                if (d.op == 0) {
                    rep->reads += 1;
                } else if (d.op == 1) {
                    rep->writes += 1;
                }
                rep->makespan_ps = max_u64(rep->makespan_ps, done);
                const uint64_t lat = done - d.issue;
                add128(rep, lat);
                rep->latency_max_ps = max_u64(rep->latency_max_ps, lat);
                if (status != NULL) {
                    status[i] = (uint8_t)(ORC_MODELED | ORC_STATUS_GROUPED);
                }
                continue;
            }
            g_lead[g_n] = i;
            g_range[g_n] = d.range_id;
            g_page[g_n] = d.page;
            ++g_n;
        }
        if (d.cls == ORC_BYPASS) {
            completion[i] = d.issue;
            rep->bypass += 1;
        } else if (d.cls == ORC_UNSUPPORTED) {
            completion[i] = UINT64_MAX;
            rep->unsupported += 1;
        } else {
            const uint64_t seq = s->modeled_sequence++;
            const uint64_t key = (d.page << p->page_shift) ^
                                 ((uint64_t)d.range_id << 32) ^ d.op;
            if (p->hybrid && orc_hybrid_reference_sample(
                                 seq, p->hybrid_warmup, p->hybrid_threshold,
                                 key)) {
                rep->hybrid_sampled += 1;
                st |= 8;
            }
            uint64_t done;
            uint64_t svc_plane;
            uint64_t xfer;
            if (p->model == ORC_MODEL_FAST_EMPIRICAL) {
                /* hbf_device.cu:796-881 with time_scale 1, in ps */
                uint64_t svc_ns = 0, packed = 0;
                uint32_t run = 0;
                orc_empirical_request_service(&p->empirical, s->burst_state,
                                              d.page, d.op, &svc_ns, &packed,
                                              &run);
                s->burst_state = packed;
                const uint64_t svc = svc_ns * 1000u;
                done = max_u64(s->channel_cursor[0], d.issue) + svc;
                s->channel_cursor[0] = done;
                s->channel_busy_total[0] += svc;
                svc_plane = svc;
                xfer = svc;
            } else {
                int hit = 0;
                if (slots) {
                    hit = pagebuf_access(&s->plane_tag[(size_t)d.plane * 2],
                                         slots, d.page);
                }
                svc_plane = hit ? d.svc_hit : d.svc_miss;
                uint64_t pd;
                if (p->plane_contention) {
                    pd = max_u64(s->plane_busy[d.plane], d.issue) + svc_plane;
                    s->plane_busy[d.plane] = pd;
                } else {
                    pd = d.issue + svc_plane;
                }
                const uint64_t cd =
                    max_u64(s->channel_cursor[d.channel], d.issue) + d.xfer;
                s->channel_cursor[d.channel] = cd;
                done = max_u64(pd, cd);
                xfer = d.xfer;
                s->plane_busy_total[d.plane] += svc_plane;
                s->channel_busy_total[d.channel] += d.xfer;
                if (d.op == 0 && hit) {
                    rep->page_hits += 1;
                    st |= 4;
                }
                if (d.op != 0 && svc_plane != 0) {
                    rep->programs += 1;
                    st |= 16;
                }
            }
            completion[i] = done;
            rep->modeled += 1;
            if (d.op == 0) {
                rep->reads += 1;
            } else if (d.op == 1) {
                rep->writes += 1;
            }
            rep->makespan_ps = max_u64(rep->makespan_ps, done);
            const uint64_t lat = done - d.issue;
            add128(rep, lat);
            rep->latency_max_ps = max_u64(rep->latency_max_ps, lat);
            rep->service_sum_ps += max_u64(svc_plane, xfer);
        }
        if (status != NULL) {
            status[i] = st;
        }
    }
    return 0;
}

/* Stable bucket of a chunk's modeled records by resource (plane or channel):
 * after the call, order[start[r] .. start[r + 1]) lists the records of
 * resource r in input order.  Counting sort, one histogram per thread over
 * a contiguous part of the chunk. */
static void bucket_by_resource(const decoded* d, size_t m, uint32_t resources,
                               int by_plane, int threads, size_t* hist,
                               size_t* start, uint32_t* order)
{
    int nt_shared = 1;
#pragma omp parallel num_threads(threads)
    {
        const int nt = omp_get_num_threads();
        const int t = omp_get_thread_num();
#pragma omp single
        nt_shared = nt;
        const size_t lo = m * (size_t)t / (size_t)nt;
        const size_t hi = m * (size_t)(t + 1) / (size_t)nt;
        size_t* h = hist + (size_t)t * resources;
        memset(h, 0, resources * sizeof(size_t));
        for (size_t i = lo; i < hi; ++i) {
            if (d[i].cls == ORC_MODELED) {
                h[by_plane ? d[i].plane : d[i].channel] += 1;
            }
        }
#pragma omp barrier
#pragma omp single
        {
            size_t acc = 0;
            for (uint32_t r = 0; r < resources; ++r) {
                start[r] = acc;
                for (int u = 0; u < nt_shared; ++u) {
                    const size_t c = hist[(size_t)u * resources + r];
                    hist[(size_t)u * resources + r] = acc;
                    acc += c;
                }
            }
            start[resources] = acc;
        }
        for (size_t i = lo; i < hi; ++i) {
            if (d[i].cls == ORC_MODELED) {
                order[h[by_plane ? d[i].plane : d[i].channel]++] = (uint32_t)i;
            }
        }
    }
}

static void merge_report(orc_engine_report* t, const orc_engine_report* r)
{
    t->records += r->records;
    t->modeled += r->modeled;
    t->bypass += r->bypass;
    t->unsupported += r->unsupported;
    t->reads += r->reads;
    t->writes += r->writes;
    t->page_hits += r->page_hits;
    t->programs += r->programs;
    t->hybrid_sampled += r->hybrid_sampled;
    t->makespan_ps = max_u64(t->makespan_ps, r->makespan_ps);
    const uint64_t lo = t->latency_sum_lo + r->latency_sum_lo;
    t->latency_sum_hi += r->latency_sum_hi + (lo < t->latency_sum_lo);
    t->latency_sum_lo = lo;
    t->latency_max_ps = max_u64(t->latency_max_ps, r->latency_max_ps);
    t->service_sum_ps += r->service_sum_ps;
    t->grouped += r->grouped;
}

/* Parallel oracle, identical results to orc_engine_run for ORC_MODEL_HBF.
 * The stream is taken in chunks of 2^24 records, with engine state carried
 * from chunk to chunk exactly as from record to record.  Per chunk:
 * classification/decode in parallel over records; the records bucketed by
 * plane (stable), the plane stage in parallel over planes, each plane's
 * records in input order; the same by channel for the channel stage; then
 * status, report and the hybrid sequence in parallel over parts of the
 * chunk, each part's sequence numbers offset by the modeled records before
 * it. */
static int engine_run_parallel_in_order(const orc_engine_params* p,
                                        const orc_range* ranges, uint32_t range_count,
                                        const orc_record* records, size_t n,
                                        uint64_t base_ps, orc_engine_state* s,
                                        uint64_t* completion, uint8_t* status,
                                        orc_engine_report* rep, int threads)
{
    if (p->model != ORC_MODEL_HBF || threads <= 1 || p->warp_grouping) {
        return engine_run_in_order(p, ranges, range_count, records, n, base_ps, s,
                                   completion, status, rep);
    }
    if (!engine_params_ok(p)) {
        return 1;
    }
    const uint32_t planes = p->channels * p->ways * p->dies * p->planes;
    const uint32_t resources = planes > p->channels ? planes : p->channels;
    const uint32_t slots = p->page_buffers;
    const size_t chunk = (size_t)1 << 24;
    const size_t cap = n < chunk ? (n ? n : 1) : chunk;
    decoded* d = (decoded*)malloc(cap * sizeof(decoded));
    uint64_t* pd = (uint64_t*)malloc(cap * sizeof(uint64_t));
    uint8_t* hit = (uint8_t*)malloc(cap);
    uint32_t* order = (uint32_t*)malloc(cap * sizeof(uint32_t));
    size_t* hist = (size_t*)malloc((size_t)threads * resources * sizeof(size_t));
    size_t* start = (size_t*)malloc(((size_t)resources + 1) * sizeof(size_t));
    size_t* part_modeled = (size_t*)calloc((size_t)threads + 1, sizeof(size_t));
    orc_engine_report* part = (orc_engine_report*)calloc((size_t)threads, sizeof(orc_engine_report));
    if (!d || !pd || !hit || !order || !hist || !start || !part_modeled || !part) {
        free(d); free(pd); free(hit); free(order); free(hist); free(start);
        free(part_modeled); free(part);
        return 2;
    }
    for (size_t c0 = 0; c0 < n; c0 += cap) {
        const size_t m = n - c0 < cap ? n - c0 : cap;
        const orc_record* rec = records + c0;
        uint64_t* comp = completion + c0;
        uint8_t* stat = status != NULL ? status + c0 : NULL;
#pragma omp parallel for num_threads(threads) schedule(static)
        for (size_t i = 0; i < m; ++i) {
            decode(p, ranges, range_count, &rec[i], base_ps, &d[i]);
            hit[i] = 0;
        }
        /* plane stage */
        bucket_by_resource(d, m, planes, 1, threads, hist, start, order);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (uint32_t pl = 0; pl < planes; ++pl) {
            /* the plane's state in locals: neighbouring planes share cache
             * lines and belong to other threads */
            uint64_t tags[2] = {s->plane_tag[(size_t)pl * 2],
                                s->plane_tag[(size_t)pl * 2 + 1]};
            uint64_t busy = s->plane_busy[pl];
            uint64_t total = 0;
            for (size_t k = start[pl]; k < start[pl + 1]; ++k) {
                const size_t i = order[k];
                int h = 0;
                if (slots) {
                    h = pagebuf_access(tags, slots, d[i].page);
                }
                hit[i] = (uint8_t)h;
                const uint64_t svc = h ? d[i].svc_hit : d[i].svc_miss;
                if (p->plane_contention) {
                    busy = max_u64(busy, d[i].issue) + svc;
                    pd[i] = busy;
                } else {
                    pd[i] = d[i].issue + svc;
                }
                total += svc;
            }
            if (start[pl] != start[pl + 1]) {
                s->plane_tag[(size_t)pl * 2] = tags[0];
                s->plane_tag[(size_t)pl * 2 + 1] = tags[1];
                s->plane_busy[pl] = busy;
                s->plane_busy_total[pl] += total;
            }
        }
        /* channel stage */
        bucket_by_resource(d, m, p->channels, 0, threads, hist, start, order);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (uint32_t ch = 0; ch < p->channels; ++ch) {
            uint64_t cursor = s->channel_cursor[ch];
            uint64_t total = 0;
            for (size_t k = start[ch]; k < start[ch + 1]; ++k) {
                const size_t i = order[k];
                cursor = max_u64(cursor, d[i].issue) + d[i].xfer;
                comp[i] = max_u64(pd[i], cursor);
                total += d[i].xfer;
            }
            s->channel_cursor[ch] = cursor;
            s->channel_busy_total[ch] += total;
        }
        /* status and report: modeled counts per part, then the parts */
        int nparts = 1;
#pragma omp parallel num_threads(threads)
        {
            const int nt = omp_get_num_threads();
            const int t = omp_get_thread_num();
#pragma omp single
            nparts = nt;
            const size_t lo = m * (size_t)t / (size_t)nt;
            const size_t hi = m * (size_t)(t + 1) / (size_t)nt;
            size_t cnt = 0;
            for (size_t i = lo; i < hi; ++i) {
                cnt += d[i].cls == ORC_MODELED;
            }
            part_modeled[t + 1] = cnt;
#pragma omp barrier
#pragma omp single
            {
                part_modeled[0] = 0;
                for (int u = 0; u < nparts; ++u) {
                    part_modeled[u + 1] += part_modeled[u];
                }
            }
            orc_engine_report* r = &part[t];
            memset(r, 0, sizeof(*r));
            uint64_t seq = s->modeled_sequence + part_modeled[t];
            for (size_t i = lo; i < hi; ++i) {
                r->records += 1;
                uint8_t st = (uint8_t)d[i].cls;
                if (d[i].cls == ORC_BYPASS) {
                    comp[i] = d[i].issue;
                    r->bypass += 1;
                } else if (d[i].cls == ORC_UNSUPPORTED) {
                    comp[i] = UINT64_MAX;
                    r->unsupported += 1;
                } else {
                    const uint64_t key = (d[i].page << p->page_shift) ^
                                         ((uint64_t)d[i].range_id << 32) ^ d[i].op;
                    if (p->hybrid && orc_hybrid_reference_sample(
                                         seq, p->hybrid_warmup, p->hybrid_threshold,
                                         key)) {
                        r->hybrid_sampled += 1;
                        st |= 8;
                    }
                    ++seq;
                    const uint64_t svc = hit[i] ? d[i].svc_hit : d[i].svc_miss;
                    r->modeled += 1;
                    if (d[i].op == 0) {
                        r->reads += 1;
                        if (hit[i]) {
                            r->page_hits += 1;
                            st |= 4;
                        }
                    } else {
                        if (d[i].op == 1) {
                            r->writes += 1;
                        }
                        if (svc != 0) {
                            r->programs += 1;
                            st |= 16;
                        }
                    }
                    const uint64_t done = comp[i];
                    r->makespan_ps = max_u64(r->makespan_ps, done);
                    const uint64_t lat = done - d[i].issue;
                    add128(r, lat);
                    r->latency_max_ps = max_u64(r->latency_max_ps, lat);
                    r->service_sum_ps += max_u64(svc, d[i].xfer);
                }
                if (stat != NULL) {
                    stat[i] = st;
                }
            }
        }
        for (int u = 0; u < nparts; ++u) {
            merge_report(rep, &part[u]);
        }
        s->modeled_sequence += part_modeled[nparts];
    }
    free(d);
    free(pd);
    free(hit);
    free(order);
    free(hist);
    free(start);
    free(part_modeled);
    free(part);
    return 0;
}

/* ---- issue order ----------------------------------------------------
 * Every resource serves its records in (issue time, stream position)
 * order: the order in which the reference's MQSim adapter serves staged
 * arrivals, sorted by (arrival, sequence) (mqsim_online.cpp:269-289).  A
 * stream already in issue order is run as it lies.  Any other stream is run
 * from a copy sorted by (issue_ps, position), and its completions and
 * statuses are written back to stream positions.  Warp groups are checked
 * on the stream as given, then again on the sorted copy. */
static int issue_ordered(const orc_record* r, size_t n)
{
    for (size_t i = 1; i < n; ++i) {
        if (r[i].issue_ps < r[i - 1].issue_ps) {
            return 0;
        }
    }
    return 1;
}

/* pos[] = 0..n-1 stably merge-sorted by issue_ps (tmp: n entries). */
static void issue_sort(const orc_record* r, size_t n, size_t* pos, size_t* tmp)
{
    for (size_t i = 0; i < n; ++i) {
        pos[i] = i;
    }
    size_t* a = pos;
    size_t* b = tmp;
    for (size_t w = 1; w < n; w *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * w) {
            const size_t mid = lo + w < n ? lo + w : n;
            const size_t hi = lo + 2 * w < n ? lo + 2 * w : n;
            size_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) {
                /* ties take the left run first: stream order is kept */
                b[k++] = r[a[j]].issue_ps < r[a[i]].issue_ps ? a[j++] : a[i++];
            }
            while (i < mid) b[k++] = a[i++];
            while (j < hi) b[k++] = a[j++];
        }
        size_t* t = a;
        a = b;
        b = t;
    }
    if (a != pos) {
        memcpy(pos, a, n * sizeof(size_t));
    }
}

static int engine_run_ordered(const orc_engine_params* p, const orc_range* ranges,
                              uint32_t range_count, const orc_record* records, size_t n,
                              uint64_t base_ps, orc_engine_state* s, uint64_t* completion,
                              uint8_t* status, orc_engine_report* rep, int threads)
{
    if (issue_ordered(records, n)) {
        return engine_run_parallel_in_order(p, ranges, range_count, records, n, base_ps, s,
                                            completion, status, rep, threads);
    }
    if (!engine_params_ok(p)) {
        return 1;
    }
    if (p->warp_grouping && !groups_valid(p, records, n)) {
        return 6;
    }
    size_t* pos = (size_t*)malloc(n * sizeof(size_t));
    size_t* tmp = (size_t*)malloc(n * sizeof(size_t));
    orc_record* sorted = (orc_record*)malloc(n * sizeof(orc_record));
    uint64_t* comp = (uint64_t*)malloc(n * sizeof(uint64_t));
    uint8_t* st = (uint8_t*)malloc(n);
    int rc = 2;
    if (pos && tmp && sorted && comp && st) {
        issue_sort(records, n, pos, tmp);
        for (size_t j = 0; j < n; ++j) {
            sorted[j] = records[pos[j]];
        }
        rc = engine_run_parallel_in_order(p, ranges, range_count, sorted, n, base_ps, s, comp,
                                          st, rep, threads);
        if (rc == 0) {
            for (size_t j = 0; j < n; ++j) {
                completion[pos[j]] = comp[j];
                if (status != NULL) {
                    status[pos[j]] = st[j];
                }
            }
        }
    }
    free(pos);
    free(tmp);
    free(sorted);
    free(comp);
    free(st);
    return rc;
}

int orc_engine_run(const orc_engine_params* p, const orc_range* ranges,
                   uint32_t range_count, const orc_record* records, size_t n,
                   uint64_t base_ps, orc_engine_state* s, uint64_t* completion,
                   uint8_t* status, orc_engine_report* rep)
{
    return engine_run_ordered(p, ranges, range_count, records, n, base_ps, s, completion,
                              status, rep, 1);
}

int orc_engine_run_parallel(const orc_engine_params* p,
                            const orc_range* ranges, uint32_t range_count,
                            const orc_record* records, size_t n,
                            uint64_t base_ps, orc_engine_state* s,
                            uint64_t* completion, uint8_t* status,
                            orc_engine_report* rep, int threads)
{
    return engine_run_ordered(p, ranges, range_count, records, n, base_ps, s, completion,
                              status, rep, threads);
}

/* hbf_device.cu:883-958, time_scale 1: one global tail; the latency bound
 * and the transfer tail are independent and the target is their maximum. */
uint64_t orc_fast_model_scalar(const uint64_t* arrival_ns,
                               const uint32_t* operation, const uint32_t* bytes,
                               size_t n, uint64_t read_ns, uint64_t program_ns,
                               uint64_t bandwidth, uint64_t* tail_ns,
                               uint64_t* target_ns)
{
    uint64_t modeled = 0;
    for (size_t i = 0; i < n; ++i) {
        const uint64_t base = operation[i] == 0 ? read_ns : program_ns;
        const uint64_t xfer = orc_fast_transfer_ns(bytes[i], bandwidth);
        const uint64_t start = *tail_ns > arrival_ns[i] ? *tail_ns
                                                        : arrival_ns[i];
        const uint64_t transfer_target = orc_saturating_add(start, xfer);
        *tail_ns = transfer_target;
        const uint64_t latency_target =
            orc_saturating_add(arrival_ns[i], base);
        target_ns[i] = latency_target > transfer_target ? latency_target
                                                        : transfer_target;
        modeled += orc_fast_service_ns(base, bytes[i], bandwidth);
    }
    return modeled;
}

/* hbf_trace_timing.cpp:92-121 (event validation) and :181-233 (fast loop):
 * ordered blocking replay, clock += max(base, transfer) per page. */
int orc_trace_timing_fast(const orc_trace_event* ev, size_t n,
                          uint64_t read_ns, uint64_t program_ns,
                          uint64_t bandwidth, uint64_t profile_page_bytes,
                          uint64_t capacity_bytes, uint64_t* submitted,
                          uint64_t* service_ns, uint64_t* clock_ns)
{
    uint64_t seq = 0, clock = 0, service = 0;
    for (size_t i = 0; i < n; ++i) {
        const uint64_t bytes = ev[i].bytes;
        const uint64_t page = ev[i].page_bytes;
        if (bytes == 0 || page == 0 || bytes % page != 0 || page % 512 != 0 ||
            ev[i].operation > 1 || ev[i].logical_address % page != 0 ||
            bytes > UINT64_MAX - ev[i].logical_address) {
            return 64;
        }
        if (page != profile_page_bytes ||
            ev[i].logical_address + bytes > capacity_bytes) {
            return 64;
        }
        for (uint64_t off = 0; off < bytes; off += page) {
            ++seq;
            const uint64_t base = ev[i].operation ? program_ns : read_ns;
            const u128 t = ((u128)page * 1000000000ULL + bandwidth - 1) /
                           bandwidth;
            const uint64_t xfer = (uint64_t)t;
            const uint64_t exposed = xfer > base ? xfer : base;
            service = orc_saturating_add(service, exposed);
            clock = orc_saturating_add(clock, exposed);
        }
    }
    *submitted = seq;
    *service_ns = service;
    *clock_ns = clock;
    return 0;
}

/* mqsim_online.cpp:321-335: bandwidth cursor lower-bounds completion */
uint64_t orc_bandwidth_cursor(uint64_t* cursor_ns, uint64_t arrival_ns,
                              uint64_t bytes, uint64_t bandwidth,
                              uint64_t media_completion_ns)
{
    const uint64_t xfer = (uint64_t)(((u128)bytes * 1000000000ULL +
                                      bandwidth - 1) / bandwidth);
    *cursor_ns = max_u64(*cursor_ns, arrival_ns) + xfer;
    return max_u64(media_completion_ns, *cursor_ns);
}

/* MQSim-style event queue: (time, registration order) min-heap. */
typedef struct adm_event {
    uint64_t time, order;
    uint32_t kind;  /* 0 arrival, 1 completion */
    uint32_t request;
} adm_event;

static int adm_before(const adm_event* a, const adm_event* b)
{
    return a->time != b->time ? a->time < b->time : a->order < b->order;
}

static void adm_push(adm_event* h, size_t* size, adm_event e)
{
    size_t i = (*size)++;
    h[i] = e;
    while (i > 0 && adm_before(&h[i], &h[(i - 1) / 2])) {
        const adm_event t = h[i];
        h[i] = h[(i - 1) / 2];
        h[(i - 1) / 2] = t;
        i = (i - 1) / 2;
    }
}

static adm_event adm_pop(adm_event* h, size_t* size)
{
    const adm_event top = h[0];
    h[0] = h[--(*size)];
    size_t i = 0;
    for (;;) {
        const size_t l = 2 * i + 1, r = l + 1;
        size_t m = i;
        if (l < *size && adm_before(&h[l], &h[m])) m = l;
        if (r < *size && adm_before(&h[r], &h[m])) m = r;
        if (m == i) break;
        const adm_event t = h[i];
        h[i] = h[m];
        h[m] = t;
        i = m;
    }
    return top;
}

static const uint64_t* adm_sort_key;
static int adm_cmp(const void* pa, const void* pb)
{
    const uint32_t a = *(const uint32_t*)pa, b = *(const uint32_t*)pb;
    if (adm_sort_key[a] != adm_sort_key[b]) {
        return adm_sort_key[a] < adm_sort_key[b] ? -1 : 1;
    }
    return a < b ? -1 : (a > b);
}

int orc_mqsim_admission(const uint64_t* arrival_ns, const uint64_t* bytes,
                        const uint64_t* latency_ns, size_t n, uint32_t queue_depth,
                        uint64_t bandwidth, uint64_t* admission_ns, uint64_t* device_ns,
                        uint64_t* completion_ns)
{
    if (bandwidth == 0 || n >= ((size_t)1 << 32)) {
        return 1;
    }
    if (n == 0) {
        return 0;
    }
    const uint64_t depth = queue_depth == 0 ? 1 : queue_depth;  /* max(1, queue_depth) */
    uint32_t* staged = malloc(n * sizeof(uint32_t));
    uint32_t* fifo = malloc(n * sizeof(uint32_t));
    uint8_t* readmitted = calloc(n, 1);
    adm_event* heap = malloc(3 * n * sizeof(adm_event));  /* arrivals, completions, re-registrations */
    size_t size = 0, fhead = 0, ftail = 0;
    uint64_t order = 0, in_device = 0, cursor = 0;
    for (size_t i = 0; i < n; ++i) {
        staged[i] = (uint32_t)i;
    }
    adm_sort_key = arrival_ns;
    qsort(staged, n, sizeof(uint32_t), adm_cmp);  /* flush_staged */
    for (size_t i = 0; i < n; ++i) {
        const adm_event e = {arrival_ns[staged[i]], order++, 0, staged[i]};
        adm_push(heap, &size, e);
    }
    while (size != 0) {
        const adm_event e = adm_pop(heap, &size);
        const uint32_t k = e.request;
        if (e.kind == 0) {  /* submit_to_device */
            if (!readmitted[k]) {
                if (in_device >= depth) {
                    fifo[ftail++] = k;
                    continue;
                }
                ++in_device;
            }
            readmitted[k] = 0;
            admission_ns[k] = e.time;  /* dispatch_to_device */
            device_ns[k] = e.time + latency_ns[k];
            const adm_event c = {device_ns[k], order++, 1, k};
            adm_push(heap, &size, c);
        } else {  /* the completion callback */
            completion_ns[k] = orc_bandwidth_cursor(&cursor, arrival_ns[k], bytes[k],
                                                    bandwidth, e.time);
            --in_device;
            while (in_device < depth && fhead != ftail) {  /* release_admission_slots */
                const uint32_t j = fifo[fhead++];
                readmitted[j] = 1;
                ++in_device;
                const adm_event a = {e.time, order++, 0, j};
                adm_push(heap, &size, a);
            }
        }
    }
    free(staged);
    free(fifo);
    free(readmitted);
    free(heap);
    return 0;
}

/* The adapter's admission and bandwidth cursor (mqsim_online.cpp:269-376)
 * with this engine as the media port, as one event loop: request k's pages
 * are records[first[k] .. first[k + 1]); when the loop dispatches it (at its
 * arrival, or at the completion that frees its slot) the engine times its
 * pages issued at that time, with the engine state carried from the requests
 * dispatched before it, and its device completion (ns, the ceiling of the
 * engine's latest page completion) is an event like MQSim's completion
 * callback.  Times in ns as the adapter's; issue_ps = dispatch ns * 1000. */
int orc_engine_admission(const orc_engine_params* p, const orc_range* ranges,
                         uint32_t range_count, const orc_record* records,
                         const uint64_t* first, size_t n, const uint64_t* arrival_ns,
                         const uint64_t* bytes, uint32_t queue_depth, uint64_t bandwidth,
                         orc_engine_state* s, uint64_t* admission_ns, uint64_t* device_ns,
                         uint64_t* completion_ns)
{
    if (bandwidth == 0 || n >= ((size_t)1 << 32)) {
        return 1;
    }
    if (n == 0) {
        return 0;
    }
    const uint64_t depth = queue_depth == 0 ? 1 : queue_depth;
    size_t most = 1;
    for (size_t k = 0; k < n; ++k) {
        const size_t m = (size_t)(first[k + 1] - first[k]);
        most = m > most ? m : most;
    }
    uint32_t* staged = malloc(n * sizeof(uint32_t));
    uint32_t* fifo = malloc(n * sizeof(uint32_t));
    uint8_t* readmitted = calloc(n, 1);
    adm_event* heap = malloc(3 * n * sizeof(adm_event));
    orc_record* pages = malloc(most * sizeof(orc_record));
    uint64_t* done = malloc(most * sizeof(uint64_t));
    int rc = 0;
    if (!staged || !fifo || !readmitted || !heap || !pages || !done) {
        rc = 2;
        goto out;
    }
    size_t size = 0, fhead = 0, ftail = 0;
    uint64_t order = 0, in_device = 0, cursor = 0;
    for (size_t i = 0; i < n; ++i) {
        staged[i] = (uint32_t)i;
    }
    adm_sort_key = arrival_ns;
    qsort(staged, n, sizeof(uint32_t), adm_cmp);  /* flush_staged */
    for (size_t i = 0; i < n; ++i) {
        const adm_event e = {arrival_ns[staged[i]], order++, 0, staged[i]};
        adm_push(heap, &size, e);
    }
    while (size != 0) {
        const adm_event e = adm_pop(heap, &size);
        const uint32_t k = e.request;
        if (e.kind == 0) {  /* submit_to_device */
            if (!readmitted[k]) {
                if (in_device >= depth) {
                    fifo[ftail++] = k;
                    continue;
                }
                ++in_device;
            }
            readmitted[k] = 0;
            admission_ns[k] = e.time;  /* dispatch_to_device: the engine times the pages */
            const size_t b = (size_t)first[k], m = (size_t)(first[k + 1] - first[k]);
            for (size_t j = 0; j < m; ++j) {
                pages[j] = records[b + j];
                pages[j].issue_ps = e.time * 1000u;
            }
            orc_engine_report rep;
            memset(&rep, 0, sizeof(rep));
            rc = orc_engine_run(p, ranges, range_count, pages, m, 0, s, done, NULL, &rep);
            if (rc != 0) {
                goto out;
            }
            uint64_t last = e.time * 1000u;
            for (size_t j = 0; j < m; ++j) {
                last = done[j] > last ? done[j] : last;
            }
            device_ns[k] = (last + 999) / 1000;
            const adm_event c = {device_ns[k], order++, 1, k};
            adm_push(heap, &size, c);
        } else {  /* the completion callback */
            completion_ns[k] = orc_bandwidth_cursor(&cursor, arrival_ns[k], bytes[k],
                                                    bandwidth, e.time);
            --in_device;
            while (in_device < depth && fhead != ftail) {  /* release_admission_slots */
                const uint32_t j = fifo[fhead++];
                readmitted[j] = 1;
                ++in_device;
                const adm_event a = {e.time, order++, 0, j};
                adm_push(heap, &size, a);
            }
        }
    }
out:
    free(staged);
    free(fifo);
    free(readmitted);
    free(heap);
    free(pages);
    free(done);
    return rc;
}

/* prefetch_model.cpp:22-50: k identical servers; a read issued at `now`
 * takes the server that frees first and finishes one latency later. */
/* MediaServers::issue (prefetch_model.cpp:37-46): the server that frees
 * first takes the read.  The servers are identical, so a scan for the
 * minimum free-at time serves as the heap. */
static uint64_t servers_issue(uint64_t* free_at, uint32_t k, uint64_t now, uint64_t latency)
{
    uint32_t best = 0;
    for (uint32_t j = 1; j < k; ++j) {
        if (free_at[j] < free_at[best]) {
            best = j;
        }
    }
    const uint64_t start = max_u64(now, free_at[best]);
    free_at[best] = start + latency;
    return free_at[best];
}

void orc_media_servers(const uint64_t* now_ns, size_t n, uint32_t servers,
                       uint64_t latency_ns, uint64_t* completion_ns)
{
    const uint32_t k = servers ? servers : 1;
    uint64_t* free_at = (uint64_t*)calloc(k, sizeof(uint64_t));
    if (free_at == NULL) {
        return;
    }
    for (size_t i = 0; i < n; ++i) {
        completion_ns[i] = servers_issue(free_at, k, now_ns[i], latency_ns);
    }
    free(free_at);
}

/* StagingBuffer (prefetch_model.cpp:55-103): pages in insertion order with
 * their arrival times; inserting past the capacity drops the oldest. */
typedef struct {
    uint64_t* page;
    uint64_t* arrival;
    size_t size, capacity;
} staging;

static long staging_find(const staging* b, uint64_t page)
{
    for (size_t i = 0; i < b->size; ++i) {
        if (b->page[i] == page) {
            return (long)i;
        }
    }
    return -1;
}

static void staging_remove(staging* b, size_t at)
{
    for (size_t i = at + 1; i < b->size; ++i) {
        b->page[i - 1] = b->page[i];
        b->arrival[i - 1] = b->arrival[i];
    }
    --b->size;
}

int orc_simulate_prefetch(const uint64_t* pages, size_t n, uint32_t policy,
                          uint32_t lead_distance, uint32_t buffer_pages,
                          uint32_t max_in_flight, uint64_t read_latency_ns,
                          uint64_t compute_ns_per_access, uint64_t* stats)
{
    memset(stats, 0, 7 * sizeof(uint64_t));
    if (policy > 1) {
        return 1;
    }
    stats[2] = n;
    if (n == 0) {
        return 0;
    }
    const uint32_t k = max_in_flight ? max_in_flight : 1;
    staging b;
    b.capacity = buffer_pages ? buffer_pages : 1;
    b.size = 0;
    uint64_t* free_at = (uint64_t*)calloc(k, sizeof(uint64_t));
    b.page = (uint64_t*)malloc((b.capacity + 1) * sizeof(uint64_t));
    b.arrival = (uint64_t*)malloc((b.capacity + 1) * sizeof(uint64_t));
    if (!free_at || !b.page || !b.arrival) {
        free(free_at);
        free(b.page);
        free(b.arrival);
        return 1;
    }
    uint64_t clock = 0;
    for (size_t i = 0; i < n; ++i) {
        clock += compute_ns_per_access;
        /* NextPage predicts the page after this one (no workload model) */
        if (policy == 1 && lead_distance > 0) {
            const uint64_t predicted = pages[i] + 1;
            if (staging_find(&b, predicted) < 0) {
                const uint64_t arrival = servers_issue(free_at, k, clock, read_latency_ns);
                b.page[b.size] = predicted;
                b.arrival[b.size] = arrival;
                ++b.size;
                while (b.size > b.capacity) {
                    staging_remove(&b, 0);
                    ++stats[6];
                }
                ++stats[5];
            }
        }
        const long at = staging_find(&b, pages[i]);
        if (at >= 0) {
            const uint64_t arrival = b.arrival[at];
            staging_remove(&b, (size_t)at);
            ++stats[4];
            if (arrival > clock) {
                stats[1] += arrival - clock;
                clock = arrival;
            }
        } else {
            const uint64_t arrival = servers_issue(free_at, k, clock, read_latency_ns);
            ++stats[3];
            stats[1] += arrival - clock;
            clock = arrival;
        }
    }
    stats[6] += b.size;
    stats[0] = clock;
    free(free_at);
    free(b.page);
    free(b.arrival);
    return 0;
}

/* ---- thermal: thermal.cpp:172-193 (matrix), 127-160 (Cholesky), 242-311
 * (backward-Euler step with constant segment power) -------------------- */
int orc_thermal_dense_step(size_t n, const double* capacity,
                           const double* boundary_g, const double* boundary_t,
                           const double* static_power, size_t n_edges,
                           const uint32_t* edge_a, const uint32_t* edge_b,
                           const double* edge_g, double dt,
                           const double* energy, double* temperature)
{
    double* a = (double*)calloc(n * n, sizeof(double));
    double* l = (double*)calloc(n * n, sizeof(double));
    double* rhs = (double*)malloc(n * sizeof(double));
    double* y = (double*)malloc(n * sizeof(double));
    int rc = 0;
    if (!a || !l || !rhs || !y) {
        rc = 2;
        goto out;
    }
    for (size_t i = 0; i < n; ++i) {
        a[i * n + i] = capacity[i] / dt + boundary_g[i];
    }
    for (size_t e = 0; e < n_edges; ++e) {
        const size_t i = edge_a[e], j = edge_b[e];
        a[i * n + i] += edge_g[e];
        a[j * n + j] += edge_g[e];
        a[i * n + j] -= edge_g[e];
        a[j * n + i] -= edge_g[e];
    }
    for (size_t i = 0; i < n; ++i) {
        for (size_t j = 0; j <= i; ++j) {
            double sum = a[i * n + j];
            for (size_t k = 0; k < j; ++k) {
                sum -= l[i * n + k] * l[j * n + k];
            }
            if (i == j) {
                if (!(sum > 0.0)) {
                    rc = 1;
                    goto out;
                }
                l[i * n + j] = sqrt(sum);
            } else {
                l[i * n + j] = sum / l[j * n + j];
            }
        }
    }
    for (size_t i = 0; i < n; ++i) {
        rhs[i] = capacity[i] / dt * temperature[i] + static_power[i] +
                 (energy ? energy[i] : 0.0) / dt +
                 boundary_g[i] * boundary_t[i];
    }
    for (size_t i = 0; i < n; ++i) {
        double sum = rhs[i];
        for (size_t j = 0; j < i; ++j) {
            sum -= l[i * n + j] * y[j];
        }
        y[i] = sum / l[i * n + i];
    }
    for (size_t i = n; i-- > 0;) {
        double sum = y[i];
        for (size_t j = i + 1; j < n; ++j) {
            sum -= l[j * n + i] * temperature[j];
        }
        temperature[i] = sum / l[i * n + i];
    }
out:
    free(a);
    free(l);
    free(rhs);
    free(y);
    return rc;
}

/* The same backward-Euler step on a regular grid, solved by Jacobi sweeps:
 * T_i <- (C/dt T_i^old + P_i + sum_j g_ij T_j + gb_i tb) / (C/dt + sum_j g_ij
 * + gb_i).  Converges because the system is strictly diagonally dominant. */
/* Jacobi sweeps over caller-provided buffers (old = T at the start of the
 * step, cur = current iterate, nxt = scratch).  Each cell's numerator and
 * denominator are accumulated in a fixed order -- x-1, x+1, y-1, y+1, z-1,
 * z+1, ambient -- and the update is num * (1 / den); the GPU stencil
 * follows this operation for operation. */
static int grid_jacobi(uint32_t nx, uint32_t ny, uint32_t nz, double cdt,
                       double gx, double gy, double gz, double gb, double tb,
                       const double* power, const double* old, double** curp,
                       double** nxtp, double tol, int max_sweeps)
{
    double* cur = *curp;
    double* nxt = *nxtp;
    int sweep = 0;
    for (; sweep < max_sweeps; ++sweep) {
        double delta = 0.0;
        /* every cell is computed on its own, so rows run in parallel with
         * the same results */
#pragma omp parallel for collapse(2) reduction(max : delta) schedule(static) \
    if ((size_t)nx * ny * nz >= 16384)
        for (uint32_t z = 0; z < nz; ++z) {
            for (uint32_t y = 0; y < ny; ++y) {
                for (uint32_t x = 0; x < nx; ++x) {
                    const size_t i = ((size_t)z * ny + y) * nx + x;
                    double num = cdt * old[i] + power[i];
                    double den = cdt;
                    if (x > 0) { num += gx * cur[i - 1]; den += gx; }
                    if (x + 1 < nx) { num += gx * cur[i + 1]; den += gx; }
                    if (y > 0) { num += gy * cur[i - nx]; den += gy; }
                    if (y + 1 < ny) { num += gy * cur[i + nx]; den += gy; }
                    if (z > 0) { num += gz * cur[i - (size_t)nx * ny]; den += gz; }
                    if (z + 1 < nz) { num += gz * cur[i + (size_t)nx * ny]; den += gz; }
                    if (z + 1 == nz) { num += gb * tb; den += gb; }
                    nxt[i] = num * (1.0 / den);
                    const double dd = fabs(nxt[i] - cur[i]);
                    if (dd > delta) {
                        delta = dd;
                    }
                }
            }
        }
        double* t = cur;
        cur = nxt;
        nxt = t;
        if (delta <= tol) {
            ++sweep;
            break;
        }
    }
    *curp = cur;
    *nxtp = nxt;
    return sweep;
}

int orc_thermal_grid_step(uint32_t nx, uint32_t ny, uint32_t nz,
                          double capacity, double gx, double gy, double gz,
                          double gb, double tb, double dt,
                          const double* power, double* temperature,
                          double tol, int max_sweeps)
{
    const size_t n = (size_t)nx * ny * nz;
    double* old = (double*)malloc(n * sizeof(double));
    double* cur = (double*)malloc(n * sizeof(double));
    double* nxt = (double*)malloc(n * sizeof(double));
    if (!old || !cur || !nxt) {
        free(old);
        free(cur);
        free(nxt);
        return -1;
    }
    memcpy(old, temperature, n * sizeof(double));
    memcpy(cur, temperature, n * sizeof(double));
    const int sweeps = grid_jacobi(nx, ny, nz, capacity / dt, gx, gy, gz, gb,
                                   tb, power, old, &cur, &nxt, tol, max_sweeps);
    memcpy(temperature, cur, n * sizeof(double));
    free(old);
    free(cur);
    free(nxt);
    return sweeps;
}

/* reliability.py:17-23 */
double orc_arrhenius(double temperature_k, double ea_ev, double tref_k)
{
    const double kb = 8.62e-5;
    return exp(ea_ev / kb * (1.0 / tref_k - 1.0 / temperature_k));
}

/* ---- thermal-coupled reliability ------------------------------------ */

void orc_retention_table(double ea_ev, double tref_k, uint64_t window_ps,
                         uint64_t* table)
{
    for (uint32_t b = 0; b < ORC_AF_BINS; ++b) {
        const double t = ORC_AF_T0 + ((double)b + 0.5) / ORC_AF_STEPS_PER_K;
        const double v = (double)window_ps * orc_arrhenius(t, ea_ev, tref_k);
        table[b] = v >= 1.8e19 ? UINT64_MAX : (uint64_t)llround(v);
    }
}

uint32_t orc_retention_bin(double t)
{
    if (!(t >= ORC_AF_T0)) {
        return 0;
    }
    const double f = (t - ORC_AF_T0) * ORC_AF_STEPS_PER_K;
    if (!(f < (double)(ORC_AF_BINS - 1))) {
        return ORC_AF_BINS - 1;
    }
    return (uint32_t)f;
}

static int reliability_ok(const orc_reliability* r)
{
    return r->nx && r->ny && r->nz && r->sweeps && r->regions_x &&
           r->regions_y && r->dies && r->nx % r->regions_x == 0 &&
           r->ny % r->regions_y == 0 && r->nz % r->dies == 0 &&
           r->window_ps != 0 && r->dt_s > 0.0 && r->capacity > 0.0;
}

static uint32_t die_of_cell(const orc_reliability* r, uint32_t x, uint32_t y,
                            uint32_t z)
{
    const uint32_t rw = r->nx / r->regions_x, rh = r->ny / r->regions_y;
    const uint32_t lpd = r->nz / r->dies;
    const uint32_t q = (y / rh) * r->regions_x + x / rw;
    return q * r->dies + z / lpd;
}

/* hot[d] = the hottest cell of die d (0 if none is above 0 K).  Dies are
 * disjoint blocks of cells (die_of_cell), visited in parallel. */
static void die_hotspots(const orc_reliability* r, const double* t,
                         double* hot)
{
    const uint32_t ndie = r->regions_x * r->regions_y * r->dies;
    const uint32_t rw = r->nx / r->regions_x, rh = r->ny / r->regions_y;
    const uint32_t lpd = r->nz / r->dies;
#pragma omp parallel for schedule(static) if ((size_t)r->nx * r->ny * r->nz >= 16384)
    for (uint32_t d = 0; d < ndie; ++d) {
        const uint32_t q = d / r->dies, dz = d % r->dies;
        const uint32_t x0 = (q % r->regions_x) * rw, y0 = (q / r->regions_x) * rh;
        double m = 0.0;
        for (uint32_t z = dz * lpd; z < (dz + 1) * lpd; ++z) {
            for (uint32_t y = y0; y < y0 + rh; ++y) {
                for (uint32_t x = x0; x < x0 + rw; ++x) {
                    const double v = t[((size_t)z * r->ny + y) * r->nx + x];
                    if (v > m) {
                        m = v;
                    }
                }
            }
        }
        hot[d] = m;
    }
}

/* cpu_service.cpp:221-255 (control_sample then apply_controls, policy
 * "hysteresis") for one sample at `now` with stack hotspot `hs`. */
uint32_t orc_control_step(const orc_reliability* r, orc_control* c,
                          uint64_t now, double hs)
{
    const double thr[4] = {0.0, r->light_k, r->severe_k, r->shutdown_k};
    uint32_t desired = (uint32_t)(hs >= r->light_k) +
                       (uint32_t)(hs >= r->severe_k) +
                       (uint32_t)(hs >= r->shutdown_k);
    if (desired < c->applied && hs >= thr[c->applied] - r->hysteresis_k) {
        desired = c->applied;
    }
    if (r->policy != 0) {
        if (desired == c->applied) {
            c->pending = ORC_NO_PENDING;
        } else if (c->pending == ORC_NO_PENDING || c->pending != desired) {
            const uint64_t a = orc_saturating_add(now, r->action_delay_ps);
            const uint64_t b = orc_saturating_add(c->last_change_ps, r->min_dwell_ps);
            c->pending = desired;
            c->pending_at_ps = a > b ? a : b;
        }
    }
    if (c->pending != ORC_NO_PENDING && c->pending_at_ps <= now) {
        c->applied = c->pending;
        c->last_change_ps = now;
        c->pending = ORC_NO_PENDING;
    }
    return c->applied;
}

int orc_reliability_chain(const orc_reliability* r, const uint32_t* counts,
                          uint64_t windows, double* temperature, uint64_t* age,
                          orc_control* ctl, double* hot, uint8_t* level,
                          uint8_t* refresh)
{
    if (!reliability_ok(r)) {
        return 1;
    }
    const uint32_t ndie = r->regions_x * r->regions_y * r->dies;
    const size_t n = (size_t)r->nx * r->ny * r->nz;
    const double cells =
        (double)((r->nx / r->regions_x) * (r->ny / r->regions_y) *
                 (r->nz / r->dies));
    const double pa = (r->access_energy_j / r->dt_s) / cells;
    const double pr = (r->refresh_energy_j / r->dt_s) / cells;
    const double cdt = r->capacity / r->dt_s;
    uint64_t* table = (uint64_t*)malloc(ORC_AF_BINS * sizeof(uint64_t));
    double* power = (double*)malloc(n * sizeof(double));
    double* old = (double*)malloc(n * sizeof(double));
    double* cur = (double*)malloc(n * sizeof(double));
    double* nxt = (double*)malloc(n * sizeof(double));
    if (!table || !power || !old || !cur || !nxt) {
        free(table);
        free(power);
        free(old);
        free(cur);
        free(nxt);
        return 2;
    }
    orc_retention_table(r->activation_ev, r->reference_k, r->window_ps, table);
    die_hotspots(r, temperature, hot);
    for (uint64_t w = 0; w < windows; ++w) {
        const uint64_t now = w * r->window_ps;
        const double* hp = hot + w * ndie;
        double hs = hp[0];
        for (uint32_t d = 1; d < ndie; ++d) {
            if (hp[d] > hs) {
                hs = hp[d];
            }
        }
        level[w] = (uint8_t)orc_control_step(r, ctl, now, hs);
        uint8_t* rf = refresh + w * ndie;
        for (uint32_t d = 0; d < ndie; ++d) {
            if (w > 0) {
                age[d] = orc_saturating_add(age[d], table[orc_retention_bin(hp[d])]);
            }
            rf[d] = age[d] >= r->retention_ps;
            if (rf[d]) {
                age[d] = 0;
            }
        }
        const uint32_t* cw = counts + w * ndie;
        for (uint32_t z = 0; z < r->nz; ++z) {
            for (uint32_t y = 0; y < r->ny; ++y) {
                for (uint32_t x = 0; x < r->nx; ++x) {
                    const uint32_t d = die_of_cell(r, x, y, z);
                    power[((size_t)z * r->ny + y) * r->nx + x] =
                        (r->static_w + (double)cw[d] * pa) + (double)rf[d] * pr;
                }
            }
        }
        memcpy(old, temperature, n * sizeof(double));
        memcpy(cur, temperature, n * sizeof(double));
        (void)grid_jacobi(r->nx, r->ny, r->nz, cdt, r->gx, r->gy, r->gz, r->gb,
                          r->ambient_k, power, old, &cur, &nxt, -1.0,
                          (int)r->sweeps);
        memcpy(temperature, cur, n * sizeof(double));
        die_hotspots(r, temperature, hot + (w + 1) * ndie);
    }
    free(table);
    free(power);
    free(old);
    free(cur);
    free(nxt);
    return 0;
}

uint64_t orc_defer(const uint8_t* level, uint64_t windows, uint64_t window_ps,
                   uint64_t t, uint32_t limit)
{
    uint64_t w = t / window_ps;
    if (w >= windows || level[w] < limit) {
        return t;
    }
    ++w;
    while (w < windows && level[w] >= limit) {
        ++w;
    }
    return w * window_ps;
}

void orc_admit(const uint8_t* level, uint64_t windows, uint64_t window_ps,
               uint64_t light_gap_ps, const orc_record* rec, size_t n,
               uint64_t* admit)
{
    uint64_t gate = 0;
    for (size_t i = 0; i < n; ++i) {
        const uint64_t e = orc_defer(level, windows, window_ps, rec[i].issue_ps, 2);
        const uint64_t we = e / window_ps;
        const uint64_t gap = (we < windows && level[we] == 1) ? light_gap_ps : 0;
        const uint64_t a = e > gate ? e : gate;
        admit[i] = a;
        gate = a + gap;
    }
}

size_t orc_refresh_records(const orc_engine_params* p, const uint8_t* refresh,
                           const uint8_t* level, uint64_t windows,
                           uint64_t window_ps, uint64_t* ordinal,
                           orc_record* out)
{
    const uint32_t sizes[4] = {p->channels, p->ways, p->dies, p->planes};
    uint64_t div[4];
    uint64_t stride = 1;
    for (int i = 0; i < 4; ++i) {
        div[p->order[i]] = stride;
        stride *= sizes[p->order[i]];
    }
    uint64_t rows = p->media_pages / stride;
    if (rows == 0) {
        rows = 1;
    }
    const uint32_t ndie = p->channels * p->ways * p->dies;
    size_t r = 0;
    for (uint64_t w = 0; w < windows; ++w) {
        for (uint32_t d = 0; d < ndie; ++d) {
            if (!refresh[w * ndie + d]) {
                continue;
            }
            const uint32_t q = d / p->dies, dd = d % p->dies;
            const uint64_t k = ordinal[d]++;
            const uint32_t coord[4] = {q / p->ways, q % p->ways, dd,
                                       (uint32_t)(k % p->planes)};
            uint64_t page = ((k / p->planes) % rows) * stride;
            for (int ax = 0; ax < 4; ++ax) {
                page += coord[ax] * div[ax];
            }
            out[r].addr = page;
            out[r].bytes = 2ULL << p->page_shift;
            out[r].issue_ps = orc_defer(level, windows, window_ps, w * window_ps, 3);
            out[r].flags = ORC_OP_REFRESH | ORC_FLAG_MEDIA;
            ++r;
        }
    }
    return r;
}

void orc_merge_records(const orc_record* demand, const uint64_t* admit,
                       size_t n, const orc_record* extra, size_t r,
                       orc_record* out, uint64_t* demand_pos)
{
    size_t i = 0, j = 0, k = 0;
    while (i < n || j < r) {
        if (j < r && (i == n || extra[j].issue_ps <= admit[i])) {
            out[k++] = extra[j++];
        } else {
            out[k] = demand[i];
            out[k].issue_ps = admit[i];
            demand_pos[i++] = k++;
        }
    }
}

int orc_window_counts(const orc_engine_params* p, const orc_range* ranges,
                      uint32_t range_count, const orc_record* rec, size_t n,
                      uint64_t window_ps, uint64_t windows, uint32_t* counts)
{
    if (!engine_params_ok(p) || window_ps == 0) {
        return 1;
    }
#pragma omp parallel for schedule(static) if (n >= 65536)
    for (size_t i = 0; i < n; ++i) {
        decoded d;
        decode(p, ranges, range_count, &rec[i], 0, &d);
        const uint64_t w = rec[i].issue_ps / window_ps;
        if (d.cls != ORC_MODELED || w >= windows) {
            continue;
        }
#pragma omp atomic
        counts[w * (p->channels * p->ways * p->dies) + d.plane / p->planes] += 1;
    }
    return 0;
}

void orc_set_threads(int threads)
{
    omp_set_num_threads(threads > 0 ? threads : 1);
}

int orc_get_threads(void)
{
    return omp_get_max_threads();
}

int orc_coupled_run(const orc_engine_params* p, const orc_range* ranges,
                    uint32_t range_count, const orc_reliability* r,
                    const orc_record* rec, size_t n, double* temperature,
                    uint64_t* age, orc_engine_state* s, uint64_t* completion,
                    orc_coupled_report* rep, double* hot, uint8_t* level,
                    uint8_t* refresh, uint64_t windows_cap)
{
    memset(rep, 0, sizeof(*rep));
    const uint32_t ndie = p->channels * p->ways * p->dies;
    if (!reliability_ok(r) || r->regions_x * r->regions_y != p->channels * p->ways ||
        r->dies != p->dies || p->model != ORC_MODEL_HBF) {
        return 1;
    }
    if (!issue_ordered(rec, n)) {
        return 1;  /* the windows, the admission gate and the merge follow issue order */
    }
    const uint64_t last = n ? rec[n - 1].issue_ps : 0;
    const uint64_t windows = n ? last / r->window_ps + 1 : 0;
    rep->windows = windows;
    if (windows > windows_cap) {
        return 3;
    }
    uint32_t* counts = (uint32_t*)calloc(windows * ndie + 1, sizeof(uint32_t));
    uint64_t* admit = (uint64_t*)malloc((n + 1) * sizeof(uint64_t));
    if (!counts || !admit) {
        free(counts);
        free(admit);
        return 2;
    }
    int rc = orc_window_counts(p, ranges, range_count, rec, n, r->window_ps, windows, counts);
    orc_control ctl = {0, ORC_NO_PENDING, 0, 0};
    if (rc == 0) {
        rc = orc_reliability_chain(r, counts, windows, temperature, age, &ctl, hot,
                                   level, refresh);
    }
    free(counts);
    if (rc != 0) {
        free(admit);
        return rc;
    }
    size_t nref = 0;
    for (uint64_t k = 0; k < windows * ndie; ++k) {
        nref += refresh[k];
    }
    for (uint64_t w = 0; w < windows; ++w) {
        rep->level_windows[level[w]] += 1;
    }
    for (uint64_t k = 0; k < (windows + 1) * ndie; ++k) {
        if (hot[k] > rep->peak_k) {
            rep->peak_k = hot[k];
        }
    }
    orc_admit(level, windows, r->window_ps, r->light_gap_ps, rec, n, admit);
    orc_record* extra = (orc_record*)malloc((nref + 1) * sizeof(orc_record));
    uint64_t* ordinal = (uint64_t*)calloc(ndie, sizeof(uint64_t));
    orc_record* merged = (orc_record*)malloc((n + nref + 1) * sizeof(orc_record));
    uint64_t* pos = (uint64_t*)malloc((n + 1) * sizeof(uint64_t));
    uint64_t* mcomp = (uint64_t*)malloc((n + nref + 1) * sizeof(uint64_t));
    uint8_t* mstat = (uint8_t*)malloc(n + nref + 1);
    if (!extra || !ordinal || !merged || !pos || !mcomp || !mstat) {
        rc = 2;
    } else {
        const size_t got = orc_refresh_records(p, refresh, level, windows, r->window_ps,
                                               ordinal, extra);
        (void)got;
        orc_merge_records(rec, admit, n, extra, nref, merged, pos);
        orc_engine_report er;
        memset(&er, 0, sizeof(er));
        orc_engine_params q = *p;
        q.media_records = nref != 0;
        rc = orc_engine_run_parallel(&q, ranges, range_count, merged, n + nref, 0, s, mcomp,
                                     mstat, &er, omp_get_max_threads());
        rep->refreshes = nref;
        rep->makespan_ps = er.makespan_ps;
        for (size_t i = 0; rc == 0 && i < n; ++i) {
            const uint64_t c = mcomp[pos[i]];
            completion[i] = c;
            if (admit[i] > rec[i].issue_ps) {
                rep->deferred += 1;
            }
            if ((mstat[pos[i]] & 3u) == ORC_MODELED) {
                const uint64_t lat = c - rec[i].issue_ps;
                const uint64_t lo = rep->latency_sum_lo + lat;
                rep->latency_sum_hi += lo < rep->latency_sum_lo;
                rep->latency_sum_lo = lo;
                if (lat > rep->latency_max_ps) {
                    rep->latency_max_ps = lat;
                }
                rep->demand_modeled += 1;
            }
        }
    }
    free(admit);
    free(extra);
    free(ordinal);
    free(merged);
    free(pos);
    free(mcomp);
    free(mstat);
    return rc;
}

/* ---- hybrid sampler and calibrator (src/hybrid/calibrator.cpp:67-138) -- */

typedef struct orc_class_item {
    orc_access_class key;
    uint64_t second;  /* index (sampler) or latency (calibrator) */
    size_t index;
} orc_class_item;

/* AccessClass's defaulted operator<=> (hybrid_model.hpp:13-20): operation,
 * bytes, queue_bucket, locality_bucket, in that order. */
static int class_cmp(const orc_access_class* a, const orc_access_class* b)
{
    if (a->operation != b->operation) return a->operation < b->operation ? -1 : 1;
    if (a->bytes != b->bytes) return a->bytes < b->bytes ? -1 : 1;
    if (a->queue_bucket != b->queue_bucket) return a->queue_bucket < b->queue_bucket ? -1 : 1;
    if (a->locality_bucket != b->locality_bucket)
        return a->locality_bucket < b->locality_bucket ? -1 : 1;
    return 0;
}

static int class_item_cmp(const void* pa, const void* pb)
{
    const orc_class_item* a = (const orc_class_item*)pa;
    const orc_class_item* b = (const orc_class_item*)pb;
    const int c = class_cmp(&a->key, &b->key);
    if (c != 0) return c;
    if (a->second != b->second) return a->second < b->second ? -1 : 1;
    return a->index < b->index ? -1 : (a->index > b->index ? 1 : 0);
}

/* HybridSampler (calibrator.cpp:67-96).  The constructor rejects a rate
 * outside [0, 1] or not finite and sets threshold = max for rate >= 1, else
 * rate * (long double)UINT64_MAX truncated.  reference(sequence, access)
 * inserts the class into the seen set and returns true for a warm-up
 * sequence, a class not seen before, or when the SplitMix64 finaliser of
 * sequence ^ seed ^ bytes<<17 ^ queue<<33 ^ locality<<49 ^ operation<<61 is
 * at most the threshold.  Over a stream the "not seen before" requests are
 * the first occurrence of each class, found here by sorting (class, index). */
int orc_sampler_run(uint32_t warmup, double sample_rate, uint64_t seed,
                    const orc_access_class* access, const uint64_t* sequence,
                    size_t n, uint8_t* flags)
{
    if (!isfinite(sample_rate) || sample_rate < 0.0 || sample_rate > 1.0) {
        return 1;
    }
    const uint64_t threshold = orc_sample_threshold(sample_rate);
    orc_class_item* items = (orc_class_item*)malloc((n ? n : 1) * sizeof(*items));
    if (items == NULL) {
        return 2;
    }
    for (size_t i = 0; i < n; ++i) {
        items[i].key = access[i];
        items[i].second = i;
        items[i].index = i;
        flags[i] = 0;
    }
    qsort(items, n, sizeof(*items), class_item_cmp);
    for (size_t j = 0; j < n; ++j) {
        if (j == 0 || class_cmp(&items[j].key, &items[j - 1].key) != 0) {
            flags[items[j].index] = 1;  /* unseen */
        }
    }
    free(items);
    for (size_t i = 0; i < n; ++i) {
        const orc_access_class* a = &access[i];
        uint64_t value = sequence[i] ^ seed;
        value ^= (uint64_t)a->bytes << 17;
        value ^= (uint64_t)a->queue_bucket << 33;
        value ^= (uint64_t)a->locality_bucket << 49;
        value ^= (uint64_t)a->operation << 61;
        if (sequence[i] < warmup || orc_fast_hash(value) <= threshold) {
            flags[i] = 1;
        }
    }
    return 0;
}

/* calibrator.cpp:20-30: the sample of rank ceil(size * num / den) (1-based),
 * clamped to the sorted range. */
static uint64_t class_percentile(const orc_class_item* sorted, size_t size,
                                 uint32_t num, uint32_t den)
{
    const unsigned __int128 rank =
        ((unsigned __int128)size * num + den - 1) / den;
    size_t index = rank == 0 ? 0 : (size_t)(rank - 1);
    if (index > size - 1) {
        index = size - 1;
    }
    return sorted[index].second;
}

/* Calibrator::observe then estimate for each class (calibrator.cpp:98-136):
 * samples of a class sorted ascending; count; mean = 128-bit sum / count;
 * p50, p95, p99 by class_percentile; log_mean = sum of log(sample) in long
 * double, in sorted order, / count; log_sigma = sqrt(sum (log - log_mean)^2
 * / count) in long double; both returned as double. */
long orc_calibrate(const orc_access_class* access, const uint64_t* latency,
                   size_t n, orc_calibration* rows)
{
    for (size_t i = 0; i < n; ++i) {
        if (latency[i] == 0) {
            return -1;
        }
    }
    orc_class_item* items = (orc_class_item*)malloc((n ? n : 1) * sizeof(*items));
    if (items == NULL) {
        return -1;
    }
    for (size_t i = 0; i < n; ++i) {
        items[i].key = access[i];
        items[i].second = latency[i];
        items[i].index = i;
    }
    qsort(items, n, sizeof(*items), class_item_cmp);
    long count = 0;
    size_t begin = 0;
    while (begin < n) {
        size_t end = begin + 1;
        while (end < n && class_cmp(&items[end].key, &items[begin].key) == 0) {
            ++end;
        }
        const orc_class_item* s = items + begin;
        const size_t size = end - begin;
        unsigned __int128 sum = 0;
        long double log_sum = 0.0L;
        for (size_t k = 0; k < size; ++k) {
            sum += s[k].second;
            log_sum += logl((long double)s[k].second);
        }
        const long double log_mean = log_sum / size;
        long double squared = 0.0L;
        for (size_t k = 0; k < size; ++k) {
            const long double delta = logl((long double)s[k].second) - log_mean;
            squared += delta * delta;
        }
        orc_calibration* r = &rows[count++];
        r->access = s[0].key;
        r->count = size;
        r->mean_ns = (uint64_t)(sum / size);
        r->p50_ns = class_percentile(s, size, 50, 100);
        r->p95_ns = class_percentile(s, size, 95, 100);
        r->p99_ns = class_percentile(s, size, 99, 100);
        r->log_mean = (double)log_mean;
        r->log_sigma = (double)sqrtl(squared / size);
        begin = end;
    }
    free(items);
    return count;
}
