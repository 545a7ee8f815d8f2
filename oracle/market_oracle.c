/*
 * market_oracle.c -- CPU oracle for the VecMarket matching path.
 *
 * TEST INFRASTRUCTURE ONLY (see market_oracle.h). A restatement, in plain C,
 * of the per-market logic of the reference CUDA kernels in
 * nlyu1/astra-cuda src/order_matching/market.cu. Each function cites the
 * reference lines it follows. The reference's own algorithm is kept as is
 * (including its O(L) best-price rescans), so this is also a fair CPU baseline
 * of that algorithm.
 *
 * Arithmetic: every int32 add/sub/mul that can overflow is done in uint32 and
 * cast back, i.e. two's-complement wrap, which is what the device does.
 *
 * Behaviour the reference leaves undefined (it indexes out of bounds) and that
 * this build defines identically in the oracle and on the GPU -- "parity
 * unpinned", no configuration generates these inputs:
 *   - a negative price is not inserted (reference: writes before the row,
 *     market.cu:44,58,73,87);
 *   - a negative customer id does not touch the portfolios (reference:
 *     market.cu:221-231 only checks "< num_customers");
 *   - ToString stops walking a level after max_orders nodes (reference: loops
 *     forever on a self-linked slot, market.cu:630-641).
 *
 * Parity pins for this file (tests/test_oracle_*.py): the reference's
 * pytest known-answer tests (src/tests/integration/test_vec_market.py), the
 * C++ scenario tests that agree with market.cu
 * (src/tests/unit_tests/market_tests.cu), hand-derived traces of eviction
 * aliasing and fill overflow, conservation and uncrossed-book invariants, and
 * an independently written pure-Python simulator on small random books.
 * om_clear_quotes: a cleared market behaves from then on like a fresh book with
 * the same TID counter (fills, BBOs, text, portfolio deltas) through ring
 * wrap-arounds, its heads, tails and ring position equal a fresh book's, and
 * the markets not selected go on as without the clear. om_clone: the copy
 * evolves exactly like its source, every state array equal after every step,
 * and independently of it. Each check is shown to catch planted mistakes
 * (tests/test_oracle_clear_clone.py). No function here is left unpinned.
 */
#include "market_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
static inline int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz);
    if (!p) {
        fprintf(stderr, "market_oracle: out of host memory\n");
        abort();
    }
    return p;
}

static void fill_i32(int32_t *p, size_t n, int32_t v) {
    for (size_t i = 0; i < n; ++i) p[i] = v;
}

/* Constructor state, market.cu:361-380: heads/tails/next = NULL, pool = 0,
 * slot counters = 0, portfolios = 0, host TID counter = 0 (:334). */
om_market *om_create(int32_t M, int32_t L, int32_t O, int32_t F, int32_t C) {
    om_market *mk = (om_market *)xcalloc(1, sizeof(om_market));
    size_t ml = (size_t)M * (size_t)L, mo = (size_t)M * (size_t)O;
    mk->num_markets = M;
    mk->max_price_levels = L;
    mk->max_orders = O;
    mk->max_fills = F;
    mk->num_customers = C;
    mk->global_tid = 0;
    mk->bid_heads = (int32_t *)xcalloc(ml, 4);
    mk->ask_heads = (int32_t *)xcalloc(ml, 4);
    mk->bid_tails = (int32_t *)xcalloc(ml, 4);
    mk->ask_tails = (int32_t *)xcalloc(ml, 4);
    fill_i32(mk->bid_heads, ml, OM_NULL_INDEX);
    fill_i32(mk->ask_heads, ml, OM_NULL_INDEX);
    fill_i32(mk->bid_tails, ml, OM_NULL_INDEX);
    fill_i32(mk->ask_tails, ml, OM_NULL_INDEX);
    mk->order_prices = (int32_t *)xcalloc(mo, 4);
    mk->order_sizes = (int32_t *)xcalloc(mo, 4);
    mk->order_customer_ids = (int32_t *)xcalloc(mo, 4);
    mk->order_tid = (int32_t *)xcalloc(mo, 4);
    mk->order_is_bid = (uint8_t *)xcalloc(mo, 1);
    mk->order_next = (int32_t *)xcalloc(mo, 4);
    fill_i32(mk->order_next, mo, OM_NULL_INDEX);
    mk->order_next_slots = (int32_t *)xcalloc((size_t)M, 4);
    mk->customer_portfolios = (int32_t *)xcalloc((size_t)M * (size_t)C * 2, 4);
    return mk;
}

/* Copy constructor, market.cu:385-411: every tensor cloned, TID copied. */
om_market *om_clone(const om_market *src) {
    om_market *mk = om_create(src->num_markets, src->max_price_levels, src->max_orders,
                              src->max_fills, src->num_customers);
    size_t ml = (size_t)src->num_markets * (size_t)src->max_price_levels;
    size_t mo = (size_t)src->num_markets * (size_t)src->max_orders;
    size_t mc = (size_t)src->num_markets * (size_t)src->num_customers * 2;
    mk->global_tid = src->global_tid;
    memcpy(mk->bid_heads, src->bid_heads, ml * 4);
    memcpy(mk->ask_heads, src->ask_heads, ml * 4);
    memcpy(mk->bid_tails, src->bid_tails, ml * 4);
    memcpy(mk->ask_tails, src->ask_tails, ml * 4);
    memcpy(mk->order_prices, src->order_prices, mo * 4);
    memcpy(mk->order_sizes, src->order_sizes, mo * 4);
    memcpy(mk->order_customer_ids, src->order_customer_ids, mo * 4);
    memcpy(mk->order_tid, src->order_tid, mo * 4);
    memcpy(mk->order_is_bid, src->order_is_bid, mo);
    memcpy(mk->order_next, src->order_next, mo * 4);
    memcpy(mk->order_next_slots, src->order_next_slots, (size_t)src->num_markets * 4);
    memcpy(mk->customer_portfolios, src->customer_portfolios, mc * 4);
    return mk;
}

void om_destroy(om_market *mk) {
    if (!mk) return;
    free(mk->bid_heads);
    free(mk->ask_heads);
    free(mk->bid_tails);
    free(mk->ask_tails);
    free(mk->order_prices);
    free(mk->order_sizes);
    free(mk->order_customer_ids);
    free(mk->order_tid);
    free(mk->order_is_bid);
    free(mk->order_next);
    free(mk->order_next_slots);
    free(mk->customer_portfolios);
    free(mk);
}

/* One side of add_orders_kernel: the bid block market.cu:44-70 and the ask
 * block :73-99 are the same steps on different arrays. Returns 1 if the order
 * was accepted. The slot that is reused is never unlinked from the list it was
 * on before (the reference does not do it either). */
static int om_insert(om_market *mk, int64_t m, int32_t *heads, int32_t *tails, int32_t price,
                     int32_t size, int32_t customer, int32_t tid, uint8_t is_bid) {
    const int32_t L = mk->max_price_levels, O = mk->max_orders;
    if (!(size > 0 && price < L)) return 0; /* :44 / :73 */
    if (price < 0) return 0;                /* defined here; reference is out of bounds */
    int32_t counter = mk->order_next_slots[m];        /* :46 / :75 */
    mk->order_next_slots[m] = wadd(counter, 1);
    if (counter < 0) {
        fprintf(stderr, "market_oracle: slot counter wrapped (2^31 inserts in one market)\n");
        abort();
    }
    int32_t slot = counter % O;
    int64_t idx = m * (int64_t)O + slot;               /* :47 (64-bit here) */
    mk->order_prices[idx] = price;                     /* :50-55 */
    mk->order_sizes[idx] = size;
    mk->order_customer_ids[idx] = customer;
    mk->order_tid[idx] = tid;
    mk->order_is_bid[idx] = is_bid;
    mk->order_next[idx] = OM_NULL_INDEX;
    int64_t pidx = m * (int64_t)L + price;             /* :58-69 */
    int32_t old_tail = tails[pidx];
    tails[pidx] = slot;
    if (old_tail == OM_NULL_INDEX) {
        heads[pidx] = slot;
    } else {
        mk->order_next[m * (int64_t)O + old_tail] = slot;
    }
    return 1;
}

/* Best bid: highest level with a non-NULL head, else -1 (market.cu:126-133). */
static int32_t om_scan_best_bid(const om_market *mk, int64_t m) {
    const int32_t L = mk->max_price_levels;
    for (int32_t p = L - 1; p >= 0; --p)
        if (mk->bid_heads[m * (int64_t)L + p] != OM_NULL_INDEX) return p;
    return -1;
}

/* Best ask: lowest level with a non-NULL head, else L (market.cu:135-142). */
static int32_t om_scan_best_ask(const om_market *mk, int64_t m) {
    const int32_t L = mk->max_price_levels;
    for (int32_t p = 0; p < L; ++p)
        if (mk->ask_heads[m * (int64_t)L + p] != OM_NULL_INDEX) return p;
    return L;
}

/* match_orders_kernel for one market, market.cu:117-277. */
static void om_match_market(om_market *mk, int64_t m, int32_t *fill_prices, int32_t *fill_sizes,
                            int32_t *fill_customer_ids, int32_t *fill_quoter_ids,
                            uint8_t *fill_is_sell_quote, int32_t *fill_quote_sizes,
                            int32_t *fill_tid, int32_t *fill_quote_tid, int32_t *fill_counts,
                            om_counters *cnt) {
    const int32_t L = mk->max_price_levels, O = mk->max_orders, F = mk->max_fills;
    const int32_t C = mk->num_customers;
    int32_t fill_count = 0;
    int32_t best_bid = om_scan_best_bid(mk, m);
    int32_t best_ask = om_scan_best_ask(mk, m);

    while (best_bid >= 0 && best_ask < L && best_bid >= best_ask) { /* :145-146 */
        int64_t bh = m * (int64_t)L + best_bid, ah = m * (int64_t)L + best_ask;
        int32_t bid_slot = mk->bid_heads[bh], ask_slot = mk->ask_heads[ah];
        if (bid_slot == OM_NULL_INDEX || ask_slot == OM_NULL_INDEX) break; /* :155 */
        int64_t bi = m * (int64_t)O + bid_slot, ai = m * (int64_t)O + ask_slot;
        int32_t bid_size = mk->order_sizes[bi], ask_size = mk->order_sizes[ai]; /* :161-168 */
        int32_t bid_cust = mk->order_customer_ids[bi], ask_cust = mk->order_customer_ids[ai];
        int32_t bid_tid = mk->order_tid[bi], ask_tid = mk->order_tid[ai];
        int32_t bid_price = mk->order_prices[bi], ask_price = mk->order_prices[ai];
        int bid_is_quote = bid_tid < ask_tid;                      /* :172 */
        int32_t trade_price = bid_is_quote ? bid_price : ask_price; /* :173 */
        int32_t trade_size = bid_size < ask_size ? bid_size : ask_size; /* :174 */

        if (fill_count >= F) { /* :187-195, device printf omitted */
            fill_counts[m] = -1;
            if (cnt) {
                cnt->fills += F - fill_count; /* roofline counts F for an overflow */
                cnt->overflows += 1;
            }
            return;
        }
        int64_t fi = m * (int64_t)F + fill_count; /* :198-218 */
        fill_prices[fi] = trade_price;
        fill_sizes[fi] = trade_size;
        if (bid_is_quote) {
            fill_customer_ids[fi] = ask_cust;
            fill_quoter_ids[fi] = bid_cust;
            fill_is_sell_quote[fi] = 0;
            fill_quote_sizes[fi] = bid_size;
            fill_tid[fi] = ask_tid;
            fill_quote_tid[fi] = bid_tid;
        } else {
            fill_customer_ids[fi] = bid_cust;
            fill_quoter_ids[fi] = ask_cust;
            fill_is_sell_quote[fi] = 1;
            fill_quote_sizes[fi] = ask_size;
            fill_tid[fi] = bid_tid;
            fill_quote_tid[fi] = ask_tid;
        }
        /* :221-232 (the ">= 0" halves are this build's definition) */
        if (bid_cust < C && ask_cust < C && bid_cust >= 0 && ask_cust >= 0) {
            int32_t *pb = mk->customer_portfolios + (m * (int64_t)C + bid_cust) * 2;
            int32_t *pa = mk->customer_portfolios + (m * (int64_t)C + ask_cust) * 2;
            int32_t notional = wmul(trade_price, trade_size);
            pb[0] = wadd(pb[0], trade_size);
            pb[1] = wsub(pb[1], notional);
            pa[0] = wsub(pa[0], trade_size);
            pa[1] = wadd(pa[1], notional);
        }
        fill_count++;
        if (cnt) cnt->fills += 1;

        mk->order_sizes[bi] = wsub(mk->order_sizes[bi], trade_size); /* :237-238 */
        mk->order_sizes[ai] = wsub(mk->order_sizes[ai], trade_size);

        if (mk->order_sizes[bi] == 0) { /* :241-256 */
            mk->bid_heads[bh] = mk->order_next[bi];
            if (mk->order_next[bi] == OM_NULL_INDEX) {
                mk->bid_tails[bh] = OM_NULL_INDEX;
                best_bid = om_scan_best_bid(mk, m);
                if (cnt) cnt->levels_emptied += 1;
            }
        }
        if (mk->order_sizes[ai] == 0) { /* :258-273 */
            mk->ask_heads[ah] = mk->order_next[ai];
            if (mk->order_next[ai] == OM_NULL_INDEX) {
                mk->ask_tails[ah] = OM_NULL_INDEX;
                best_ask = om_scan_best_ask(mk, m);
                if (cnt) cnt->levels_emptied += 1;
            }
        }
    }
    fill_counts[m] = fill_count; /* :277 */
}

void om_add_two_sided_quotes(om_market *mk, const int32_t *bid_px, const int32_t *bid_sz,
                             const int32_t *ask_px, const int32_t *ask_sz,
                             const int32_t *customer_ids, int32_t *fill_prices,
                             int32_t *fill_sizes, int32_t *fill_customer_ids,
                             int32_t *fill_quoter_ids, uint8_t *fill_is_sell_quote,
                             int32_t *fill_quote_sizes, int32_t *fill_tid,
                             int32_t *fill_quote_tid, int32_t *fill_counts, int nthreads,
                             om_counters *counters) {
    const int64_t M = mk->num_markets;
    const int32_t base_tid = mk->global_tid; /* :520 */
    int64_t ins = 0, fl = 0, emp = 0, ovf = 0;
    if (nthreads < 1) nthreads = 1;
    /* The reference launches add for all markets, then match for all markets
     * (:510, :549). Markets share no state, so add+match per market in one
     * pass is the same computation. fill_counts.zero_() (:543) is not needed:
     * match always writes fill_counts[m]. */
#pragma omp parallel for schedule(static) num_threads(nthreads) reduction(+ : ins, fl, emp, ovf)
    for (int64_t m = 0; m < M; ++m) {
        om_counters c = {0, 0, 0, 0};
        int32_t cust = customer_ids[m];
        c.inserts += om_insert(mk, m, mk->bid_heads, mk->bid_tails, bid_px[m], bid_sz[m], cust,
                               base_tid, 1);
        c.inserts += om_insert(mk, m, mk->ask_heads, mk->ask_tails, ask_px[m], ask_sz[m], cust,
                               wadd(base_tid, 1), 0);
        om_match_market(mk, m, fill_prices, fill_sizes, fill_customer_ids, fill_quoter_ids,
                        fill_is_sell_quote, fill_quote_sizes, fill_tid, fill_quote_tid,
                        fill_counts, &c);
        ins += c.inserts;
        fl += c.fills;
        emp += c.levels_emptied;
        ovf += c.overflows;
    }
    mk->global_tid = wadd(mk->global_tid, 2); /* :531 */
    if (counters) {
        counters->inserts = ins;
        counters->fills = fl;
        counters->levels_emptied = emp;
        counters->overflows = ovf;
    }
}

/* get_bbo_kernel, market.cu:288-319: price = best level, size = the head
 * order's remaining size; an empty side reports (NULL, 0). */
void om_get_bbos(const om_market *mk, int32_t *best_bid_prices, int32_t *best_bid_sizes,
                 int32_t *best_ask_prices, int32_t *best_ask_sizes, int nthreads) {
    const int64_t M = mk->num_markets;
    const int32_t L = mk->max_price_levels, O = mk->max_orders;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t m = 0; m < M; ++m) {
        best_bid_prices[m] = OM_NULL_INDEX;
        best_bid_sizes[m] = 0;
        best_ask_prices[m] = OM_NULL_INDEX;
        best_ask_sizes[m] = 0;
        for (int32_t p = L - 1; p >= 0; --p) {
            int32_t h = mk->bid_heads[m * (int64_t)L + p];
            if (h != OM_NULL_INDEX) {
                best_bid_prices[m] = p;
                best_bid_sizes[m] = mk->order_sizes[m * (int64_t)O + h];
                break;
            }
        }
        for (int32_t p = 0; p < L; ++p) {
            int32_t h = mk->ask_heads[m * (int64_t)L + p];
            if (h != OM_NULL_INDEX) {
                best_ask_prices[m] = p;
                best_ask_sizes[m] = mk->order_sizes[m * (int64_t)O + h];
                break;
            }
        }
    }
}

/* update_last_prices_kernel, market.cu:774-785. */
void om_update_last_prices(int32_t *last_prices, const int32_t *fill_counts,
                           const int32_t *fill_prices, int32_t num_markets, int32_t max_fills) {
    for (int64_t m = 0; m < num_markets; ++m) {
        int32_t c = fill_counts[m];
        if (c > 0) last_prices[m] = fill_prices[m * (int64_t)max_fills + (c - 1)];
    }
}

/* Reset, market.cu:699-715. The order pool itself is left as is. */
void om_reset(om_market *mk) {
    size_t ml = (size_t)mk->num_markets * (size_t)mk->max_price_levels;
    size_t mo = (size_t)mk->num_markets * (size_t)mk->max_orders;
    fill_i32(mk->bid_heads, ml, OM_NULL_INDEX);
    fill_i32(mk->ask_heads, ml, OM_NULL_INDEX);
    fill_i32(mk->bid_tails, ml, OM_NULL_INDEX);
    fill_i32(mk->ask_tails, ml, OM_NULL_INDEX);
    fill_i32(mk->order_next, mo, OM_NULL_INDEX);
    memset(mk->order_next_slots, 0, (size_t)mk->num_markets * 4);
    memset(mk->customer_portfolios, 0, (size_t)mk->num_markets * mk->num_customers * 2 * 4);
    mk->global_tid = 0;
}

/* ClearQuotes, market.cu:735-749: per selected market, levels and next
 * pointers to NULL and the slot counter to 0; portfolios and TID kept. */
void om_clear_quotes(om_market *mk, const uint8_t *reset) {
    const int32_t L = mk->max_price_levels, O = mk->max_orders;
    for (int64_t m = 0; m < mk->num_markets; ++m) {
        if (!reset[m]) continue;
        fill_i32(mk->bid_heads + m * L, (size_t)L, OM_NULL_INDEX);
        fill_i32(mk->ask_heads + m * L, (size_t)L, OM_NULL_INDEX);
        fill_i32(mk->bid_tails + m * L, (size_t)L, OM_NULL_INDEX);
        fill_i32(mk->ask_tails + m * L, (size_t)L, OM_NULL_INDEX);
        fill_i32(mk->order_next + m * (int64_t)O, (size_t)O, OM_NULL_INDEX);
        mk->order_next_slots[m] = 0;
    }
}

/* ---- ToString (market.cu:599-691) -------------------------------------- */

typedef struct {
    int32_t price, size, customer, tid;
} om_row;

typedef struct {
    char *buf;
    size_t cap, len;
} om_text;

static void om_put(om_text *t, const char *s) {
    size_t n = strlen(s);
    if (t->buf && t->cap > 0 && t->len < t->cap - 1) {
        size_t room = t->cap - 1 - t->len;
        size_t k = n < room ? n : room;
        memcpy(t->buf + t->len, s, k);
        t->buf[t->len + k] = '\0';
    }
    t->len += n;
}

static int om_sell_cmp(const void *pa, const void *pb) { /* :645-651 */
    const om_row *a = (const om_row *)pa, *b = (const om_row *)pb;
    if (a->price != b->price) return a->price > b->price ? -1 : 1;
    if (a->tid != b->tid) return a->tid < b->tid ? -1 : 1;
    return 0;
}

/* Walk one level's list from its head, keeping orders with size > 0
 * (:630-641). At most max_orders nodes are visited (see the file header). */
static void om_walk(const om_market *mk, int64_t m, int32_t head, int32_t price, om_row **rows,
                    size_t *n, size_t *cap) {
    const int32_t O = mk->max_orders;
    int32_t slot = head;
    for (int32_t visited = 0; slot != OM_NULL_INDEX && visited < O; ++visited) {
        int64_t i = m * (int64_t)O + slot;
        int32_t size = mk->order_sizes[i];
        if (size > 0) {
            if (*n == *cap) {
                *cap = *cap ? 2 * *cap : 64;
                *rows = (om_row *)realloc(*rows, *cap * sizeof(om_row));
                if (!*rows) abort();
            }
            om_row r = {price, size, mk->order_customer_ids[i], mk->order_tid[i]};
            (*rows)[(*n)++] = r;
        }
        slot = mk->order_next[i];
    }
}

size_t om_to_string(const om_market *mk, int32_t market_id, char *buf, size_t buflen) {
    om_text t = {buf, buflen, 0};
    char line[160];
    if (buf && buflen) buf[0] = '\0';
    if (market_id >= mk->num_markets || market_id < 0) { /* :602-604 */
        snprintf(line, sizeof line, "Error: Invalid market_id %d (num_markets = %d)", market_id,
                 mk->num_markets);
        om_put(&t, line);
        return t.len;
    }
    const int32_t L = mk->max_price_levels;
    int64_t m = market_id;
    om_row *sells = NULL, *buys = NULL;
    size_t ns = 0, cs = 0, nb = 0, cb = 0;
    for (int32_t p = 0; p < L; ++p) om_walk(mk, m, mk->ask_heads[m * L + p], p, &sells, &ns, &cs);
    if (ns > 1) qsort(sells, ns, sizeof(om_row), om_sell_cmp);
    for (int32_t p = L - 1; p >= 0; --p) om_walk(mk, m, mk->bid_heads[m * L + p], p, &buys, &nb, &cb);

    snprintf(line, sizeof line, "####### %zu sell orders #######\n", ns); /* :677-688 */
    om_put(&t, line);
    for (size_t i = 0; i < ns; ++i) {
        snprintf(line, sizeof line, "px %d @ sz %d   id=%d @ t=%d\n", sells[i].price, sells[i].size,
                 sells[i].customer, sells[i].tid);
        om_put(&t, line);
    }
    om_put(&t, "#############################\n");
    snprintf(line, sizeof line, "####### %zu buy orders #######\n", nb);
    om_put(&t, line);
    for (size_t i = 0; i < nb; ++i) {
        snprintf(line, sizeof line, "px %d @ sz %d   id=%d @ t=%d\n", buys[i].price, buys[i].size,
                 buys[i].customer, buys[i].tid);
        om_put(&t, line);
    }
    om_put(&t, "#############################");
    free(sells);
    free(buys);
    return t.len;
}
