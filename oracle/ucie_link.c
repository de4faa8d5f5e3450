/*
 * ucie_link.c -- CPU restatement of the reference's UCIe Streaming / AoU
 * link (src/ucie/link.cpp:1-203, include/hbfsim/ucie/link.hpp,
 * src/ucie/profile.cpp:40-67).
 *
 * TEST INFRASTRUCTURE ONLY (see hbf_oracle.h): the checker the HIP link
 * kernel is compared against.  Written from the behaviour of the cited
 * functions: one link, two directions (AR requests of 3 granules, R returns
 * of 14), a Format 6 flit of 48 AoU granules every 32 / GT ns per direction,
 * every granule of a message reserved against the sender's credits at its
 * MsgStart, credits granted back on flits of the other direction in the
 * legal AoU amounts after the receiver consumes the message.  Events at one
 * time are processed in the order they were scheduled (the reference's
 * std::multimap), then both directions try to send.
 */
#include "hbf_oracle.h"

#include <stdlib.h>
#include <string.h>

enum { EV_ARRIVAL = 0, EV_DELIVERY = 1, EV_CONSUME = 2, EV_RETRY = 3 };

typedef struct ev {
    uint64_t time;
    uint64_t seq;  /* scheduling order among equal times */
    uint32_t kind, dir;
    uint64_t id;
    uint32_t grant;
    uint32_t ncompleted;
    uint64_t completed[16]; /* a flit completes at most 48 / 3 messages */
} ev;

typedef struct msg {
    uint64_t id;
    uint32_t remaining, started, emitted;
} msg;

typedef struct awaiting {
    uint32_t dir;
    uint64_t id;
    uint64_t delivered;
} awaiting;

struct orc_link {
    orc_link_profile p;
    uint64_t now;
    uint64_t seq;
    ev* heap;
    size_t nev, capev;
    msg* queue[2];
    size_t qhead[2], qlen[2], qcap[2];
    uint64_t cursor[2];
    uint32_t credits[2];      /* sender credits: [0] AR, [1] R */
    uint32_t grant_pending[2];/* [0] AR credits to grant back, [1] R credits */
    orc_link_counters counters[2];
    orc_link_flit* flits;
    size_t nflits;
    uint64_t flits_dropped;
    awaiting* aw;
    size_t naw, capaw;
    uint64_t* active[2];
    size_t nactive[2], capactive[2];
};

#define FLIT_TRACE_LIMIT 4096

/* profile.cpp:40-61 (the fields a batch link carries) */
int orc_link_profile_valid(const orc_link_profile* p)
{
    if (p->gt_per_second != 8 && p->gt_per_second != 16 && p->gt_per_second != 32) {
        return 0;
    }
    if (p->initial_ar_granules < 3 || p->initial_r_granules < 14 ||
        p->initial_ar_granules > 65535 || p->initial_r_granules > 65535) {
        return 0;
    }
    if (p->max_accepted == 0 || p->max_accepted > 65535) {
        return 0;
    }
    return p->propagation_ns <= 1000000000ULL;
}

/* profile.cpp:63-67: 256 B per flit over x64 lanes at GT/s */
uint64_t orc_link_serialization_ns(const orc_link_profile* p)
{
    return 32u / p->gt_per_second;
}

/* link.cpp:103-110 */
uint32_t orc_link_legal_grant(uint32_t pending)
{
    if (pending == 0) {
        return 0;
    }
    if (pending < 4) {
        return 1;
    }
    uint32_t grant = 4;
    while (grant < 128 && grant * 2 <= pending) {
        grant *= 2;
    }
    return grant;
}

static int ev_less(const ev* a, const ev* b)
{
    return a->time < b->time || (a->time == b->time && a->seq < b->seq);
}

static int push_event(orc_link* l, ev e)
{
    if (l->nev == l->capev) {
        size_t cap = l->capev ? 2 * l->capev : 64;
        ev* h = (ev*)realloc(l->heap, cap * sizeof(ev));
        if (!h) return 0;
        l->heap = h;
        l->capev = cap;
    }
    e.seq = l->seq++;
    size_t i = l->nev++;
    l->heap[i] = e;
    while (i > 0) {
        size_t parent = (i - 1) / 2;
        if (!ev_less(&l->heap[i], &l->heap[parent])) break;
        ev t = l->heap[i];
        l->heap[i] = l->heap[parent];
        l->heap[parent] = t;
        i = parent;
    }
    return 1;
}

static ev pop_event(orc_link* l)
{
    ev top = l->heap[0];
    l->heap[0] = l->heap[--l->nev];
    size_t i = 0;
    for (;;) {
        size_t a = 2 * i + 1, b = a + 1, m = i;
        if (a < l->nev && ev_less(&l->heap[a], &l->heap[m])) m = a;
        if (b < l->nev && ev_less(&l->heap[b], &l->heap[m])) m = b;
        if (m == i) break;
        ev t = l->heap[i];
        l->heap[i] = l->heap[m];
        l->heap[m] = t;
        i = m;
    }
    return top;
}

static int grow(void** p, size_t* cap, size_t need, size_t elem)
{
    if (need <= *cap) return 1;
    size_t c = *cap ? *cap : 16;
    while (c < need) c *= 2;
    void* q = realloc(*p, c * elem);
    if (!q) return 0;
    *p = q;
    *cap = c;
    return 1;
}

orc_link* orc_link_create(const orc_link_profile* p)
{
    if (!orc_link_profile_valid(p)) {
        return NULL;
    }
    orc_link* l = (orc_link*)calloc(1, sizeof(orc_link));
    if (!l) return NULL;
    l->p = *p;
    l->credits[0] = p->initial_ar_granules;
    l->credits[1] = p->initial_r_granules;
    l->flits = (orc_link_flit*)calloc(FLIT_TRACE_LIMIT, sizeof(orc_link_flit));
    if (!l->flits) {
        free(l);
        return NULL;
    }
    return l;
}

void orc_link_destroy(orc_link* l)
{
    if (!l) return;
    free(l->heap);
    free(l->queue[0]);
    free(l->queue[1]);
    free(l->flits);
    free(l->aw);
    free(l->active[0]);
    free(l->active[1]);
    free(l);
}

static long find_active(const orc_link* l, uint32_t dir, uint64_t id)
{
    for (size_t i = 0; i < l->nactive[dir]; ++i) {
        if (l->active[dir][i] == id) return (long)i;
    }
    return -1;
}

/* link.cpp:38-50: 0 ok, 1 invalid argument (zero id, past ready time,
 * duplicate in-flight id), 2 capacity reached */
int orc_link_enqueue(orc_link* l, uint32_t dir, uint64_t id, uint64_t ready_ns)
{
    if (dir > 1 || id == 0 || ready_ns < l->now) return 1;
    if (find_active(l, dir, id) >= 0) return 1;
    if (l->nactive[dir] >= l->p.max_accepted) return 2;
    if (!grow((void**)&l->active[dir], &l->capactive[dir], l->nactive[dir] + 1, sizeof(uint64_t)))
        return 3;
    l->active[dir][l->nactive[dir]++] = id;
    ev e;
    memset(&e, 0, sizeof(e));
    e.time = ready_ns;
    e.kind = EV_ARRIVAL;
    e.dir = dir;
    e.id = id;
    return push_event(l, e) ? 0 : 3;
}

/* link.cpp:52-61: 0 ok, 1 not delivered / consume time moved backward */
int orc_link_consume(orc_link* l, uint32_t dir, uint64_t id, uint64_t at)
{
    for (size_t i = 0; i < l->naw; ++i) {
        if (l->aw[i].dir == dir && l->aw[i].id == id) {
            if (at < l->aw[i].delivered || at < l->now) return 1;
            l->aw[i] = l->aw[--l->naw];
            ev e;
            memset(&e, 0, sizeof(e));
            e.time = at;
            e.kind = EV_CONSUME;
            e.dir = dir;
            e.id = id;
            return push_event(l, e) ? 0 : 3;
        }
    }
    return 1;
}

int orc_link_next_event(const orc_link* l, uint64_t* t)
{
    if (l->nev == 0) return 0;
    *t = l->heap[0].time;
    return 1;
}

uint64_t orc_link_now(const orc_link* l) { return l->now; }
uint32_t orc_link_credits(const orc_link* l, uint32_t dir) { return l->credits[dir & 1]; }
const orc_link_counters* orc_link_counters_of(const orc_link* l, uint32_t dir)
{
    return &l->counters[dir & 1];
}
size_t orc_link_flit_count(const orc_link* l) { return l->nflits; }
const orc_link_flit* orc_link_flit_at(const orc_link* l, size_t i) { return &l->flits[i]; }

/* link.cpp:15-23: bounded at 2^64 - 1; the direction's flag records it */
static void add_sat(orc_link_counters* c, uint64_t* target, uint64_t amount)
{
    if (amount > UINT64_MAX - *target) {
        *target = UINT64_MAX;
        c->accounting_saturated = 1;
    } else {
        *target += amount;
    }
}

/* link.cpp:112-177 for one direction; 0 ok, 2 time overflow, 3 no memory */
static int send_ready(orc_link* l, uint32_t dir)
{
    const uint32_t other = dir ^ 1u;
    /* AR data rides the request direction and R credits ride it back;
     * grant_pending[x] holds credits of direction x to return */
    uint32_t* sender_credit = &l->credits[dir];
    uint32_t* pending = &l->grant_pending[other];
    orc_link_counters* c = &l->counters[dir];
    if (l->cursor[dir] > l->now) {
        if (l->qlen[dir] != 0 || *pending != 0) {
            ev e;
            memset(&e, 0, sizeof(e));
            e.time = l->cursor[dir];
            e.kind = EV_RETRY;
            e.dir = dir;
            if (!push_event(l, e)) return 3;
        }
        return 0;
    }
    uint32_t used = 0;
    ev delivery;
    memset(&delivery, 0, sizeof(delivery));
    orc_link_flit rec;
    memset(&rec, 0, sizeof(rec));
    const uint32_t full = dir == 0 ? 3u : 14u;
    while (l->qlen[dir] != 0 && used < 48) {
        msg* m = &l->queue[dir][l->qhead[dir]];
        if (!m->started) {
            if (*sender_credit < full) break;
            *sender_credit -= full;  /* every granule reserved at MsgStart */
            m->started = 1;
        }
        const int start = m->emitted == 0;
        const uint32_t frag = 48 - used < m->remaining ? 48 - used : m->remaining;
        orc_link_fragment* f = &rec.frag[rec.nfrag++];
        f->request_id = m->id;
        f->flit_granule = used;
        f->message_granule = m->emitted;
        f->granules = frag;
        f->msg_start = (uint8_t)start;
        f->msg_end = (uint8_t)(frag == m->remaining);
        used += frag;
        m->remaining -= frag;
        m->emitted += frag;
        if (m->remaining == 0) {
            delivery.completed[delivery.ncompleted++] = m->id;
            l->qhead[dir] += 1;
            l->qlen[dir] -= 1;
        }
    }
    const uint32_t grant = orc_link_legal_grant(*pending);
    if (used == 0 && grant == 0) return 0;
    *pending -= grant;
    const uint64_t start = l->now;
    const uint64_t ser = orc_link_serialization_ns(&l->p);
    if (start > UINT64_MAX - ser) return 2;
    l->cursor[dir] = start + ser;
    if (l->cursor[dir] > UINT64_MAX - l->p.propagation_ns) return 2;
    const uint64_t at = l->cursor[dir] + l->p.propagation_ns;
    delivery.time = at;
    delivery.kind = EV_DELIVERY;
    delivery.dir = dir;
    delivery.grant = grant;
    if (!push_event(l, delivery)) return 3;
    if (l->qlen[dir] != 0 || *pending != 0) {
        ev e;
        memset(&e, 0, sizeof(e));
        e.time = l->cursor[dir];
        e.kind = EV_RETRY;
        e.dir = dir;
        if (!push_event(l, e)) return 3;
    }
    add_sat(c, &c->flits, 1);
    add_sat(c, &c->wire_bytes, 256);
    add_sat(c, &c->ucie_header_bytes, 2);
    add_sat(c, &c->crc_position_bytes, 4);
    add_sat(c, &c->aou_header_bytes, 10);
    add_sat(c, &c->aou_message_bytes, (uint64_t)used * 5);
    add_sat(c, &c->unused_message_bytes, (uint64_t)(48 - used) * 5);
    if (used == 0) add_sat(c, &c->credit_only_flits, 1);
    if (l->nflits < FLIT_TRACE_LIMIT) {
        rec.direction = dir;
        rec.start_ns = start;
        rec.delivered_ns = at;
        rec.message_granules = used;
        rec.grant_granules = grant;
        rec.credit_only = used == 0;
        l->flits[l->nflits++] = rec;
    } else {
        l->flits_dropped += 1;
    }
    return 0;
}

/* link.cpp:179-231: 0 ok, 2 overflow, 3 logic error / no memory, 4 no
 * event.  Deliveries of this step go to out[0..*count) (cap entries). */
int orc_link_step(orc_link* l, orc_link_delivery* out, size_t cap, size_t* count)
{
    *count = 0;
    if (l->nev == 0) return 4;
    l->now = l->heap[0].time;
    while (l->nev != 0 && l->heap[0].time == l->now) {
        ev e = pop_event(l);
        if (e.kind == EV_ARRIVAL) {
            const uint32_t d = e.dir;
            if (!grow((void**)&l->queue[d], &l->qcap[d], l->qhead[d] + l->qlen[d] + 1, sizeof(msg)))
                return 3;
            msg* m = &l->queue[d][l->qhead[d] + l->qlen[d]];
            m->id = e.id;
            m->remaining = d == 0 ? 3u : 14u;
            m->started = 0;
            m->emitted = 0;
            l->qlen[d] += 1;
        } else if (e.kind == EV_DELIVERY) {
            /* credits of the direction this flit carried grants for */
            const uint32_t other = e.dir ^ 1u;
            const uint32_t maximum = other == 0 ? l->p.initial_ar_granules
                                                : l->p.initial_r_granules;
            if (e.grant > maximum - l->credits[other]) return 3;
            l->credits[other] += e.grant;
            for (uint32_t k = 0; k < e.ncompleted; ++k) {
                if (*count < cap) {
                    out[*count].direction = e.dir;
                    out[*count].request_id = e.completed[k];
                    out[*count].delivered_ns = l->now;
                }
                *count += 1;
                for (size_t i = 0; i < l->naw; ++i) {
                    if (l->aw[i].dir == e.dir && l->aw[i].id == e.completed[k]) return 3;
                }
                if (!grow((void**)&l->aw, &l->capaw, l->naw + 1, sizeof(awaiting))) return 3;
                l->aw[l->naw].dir = e.dir;
                l->aw[l->naw].id = e.completed[k];
                l->aw[l->naw].delivered = l->now;
                l->naw += 1;
            }
        } else if (e.kind == EV_CONSUME) {
            const long at = find_active(l, e.dir, e.id);
            if (at < 0) return 3;
            l->active[e.dir][at] = l->active[e.dir][--l->nactive[e.dir]];
            const uint32_t amount = e.dir == 0 ? 3u : 14u;
            if (l->grant_pending[e.dir] > 65535u - amount) return 2;
            l->grant_pending[e.dir] += amount;
        }
    }
    int rc = send_ready(l, 0);
    if (rc == 0) rc = send_ready(l, 1);
    return rc;
}

/* A caller of the link that enqueues one direction-ordered stream per
 * direction and consumes every delivery `delay[dir]` after it arrives: the
 * semantics of hbfsim_amd_link_run.  Messages are admitted in order while
 * the direction has fewer than max_accepted in flight, at the later of their
 * ready time and the time the caller finds room (after each step).
 * delivered[i] receives message i's delivery time.  0 ok, else the first
 * error a link call returned. */
int orc_link_scenario_traced(const orc_link_profile* p, const uint32_t* dir,
                             const uint64_t* ready, size_t n, const uint64_t delay[2],
                             uint64_t* delivered, orc_link_counters* counters,
                             orc_link_flit* flits, size_t flits_cap, size_t* nflits,
                             uint64_t* dropped)
{
    orc_link* l = orc_link_create(p);
    if (!l) return 1;
    size_t* order[2];
    size_t cnt[2] = {0, 0};
    order[0] = (size_t*)malloc((n + 1) * sizeof(size_t));
    order[1] = (size_t*)malloc((n + 1) * sizeof(size_t));
    orc_link_delivery* out = (orc_link_delivery*)malloc(64 * sizeof(orc_link_delivery));
    int rc = 0;
    if (!order[0] || !order[1] || !out) {
        rc = 3;
        goto done;
    }
    for (size_t i = 0; i < n; ++i) {
        const uint32_t d = dir[i] & 1u;
        order[d][cnt[d]++] = i;
    }
    size_t next[2] = {0, 0};
    size_t consumed[2] = {0, 0};  /* the caller's view: consumes it issued */
    (void)consumed;
    for (;;) {
        for (uint32_t d = 0; d < 2 && rc == 0; ++d) {
            while (next[d] < cnt[d] && l->nactive[d] < p->max_accepted) {
                const size_t i = order[d][next[d]];
                const uint64_t t = ready[i] > l->now ? ready[i] : l->now;
                rc = orc_link_enqueue(l, d, (uint64_t)i + 1, t);
                if (rc != 0) break;
                next[d] += 1;
            }
        }
        uint64_t t;
        if (rc != 0 || !orc_link_next_event(l, &t)) break;
        size_t k = 0;
        rc = orc_link_step(l, out, 64, &k);
        if (rc != 0) break;
        if (k > 64) {
            rc = 3;
            break;
        }
        for (size_t j = 0; j < k && rc == 0; ++j) {
            const size_t i = (size_t)(out[j].request_id - 1);
            delivered[i] = out[j].delivered_ns;
            const uint64_t dl = delay[out[j].direction & 1u];
            if (out[j].delivered_ns > UINT64_MAX - dl) {
                rc = 2;
                break;
            }
            rc = orc_link_consume(l, out[j].direction, out[j].request_id,
                                  out[j].delivered_ns + dl);
        }
    }
    if (counters) {
        counters[0] = l->counters[0];
        counters[1] = l->counters[1];
    }
    if (flits) {
        const size_t k = l->nflits < flits_cap ? l->nflits : flits_cap;
        memcpy(flits, l->flits, k * sizeof(orc_link_flit));
        if (nflits) *nflits = k;
    }
    if (dropped) *dropped = l->flits_dropped;
done:
    free(order[0]);
    free(order[1]);
    free(out);
    orc_link_destroy(l);
    return rc;
}

int orc_link_scenario(const orc_link_profile* p, const uint32_t* dir, const uint64_t* ready,
                      size_t n, const uint64_t delay[2], uint64_t* delivered,
                      orc_link_counters* counters)
{
    return orc_link_scenario_traced(p, dir, ready, n, delay, delivered, counters, NULL, 0, NULL,
                                    NULL);
}
