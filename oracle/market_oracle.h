/*
 * market_oracle.h -- CPU oracle for the VecMarket matching path.
 *
 * TEST INFRASTRUCTURE ONLY. This is not part of the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker (or as the timed CPU baseline). The product path never calls it.
 *
 * It restates, in plain C on host memory, the per-market semantics of the
 * reference engine nlyu1/astra-cuda src/order_matching/market.cu, keeping the
 * reference's own state layout (int32 [M,L] level heads/tails, int32 [M,O]
 * order pool, int32 [M,C,2] portfolios) so every intermediate array can be
 * compared with it. The reference's compile-time caps (market.h:56-61) are
 * lifted so the deep-book shape (L=512, O=F=4096, C=64) also runs.
 */
#ifndef ASTRA_MARKET_ORACLE_H
#define ASTRA_MARKET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OM_NULL_INDEX ((int32_t)-1) /* market.h:60 */

typedef struct om_market {
    int32_t num_markets;      /* M */
    int32_t max_price_levels; /* L */
    int32_t max_orders;       /* O */
    int32_t max_fills;        /* F */
    int32_t num_customers;    /* C */
    int32_t global_tid;       /* host TID counter, market.h:338 */
    int32_t *bid_heads, *ask_heads, *bid_tails, *ask_tails;            /* [M][L] */
    int32_t *order_prices, *order_sizes, *order_customer_ids, *order_tid; /* [M][O] */
    uint8_t *order_is_bid;                                              /* [M][O] */
    int32_t *order_next;                                                /* [M][O] */
    int32_t *order_next_slots;                                          /* [M]    */
    int32_t *customer_portfolios;                                       /* [M][C][2] */
} om_market;

/* Per-call work counters used for the algorithmic-bytes roofline. */
typedef struct om_counters {
    int64_t inserts;        /* accepted order inserts */
    int64_t fills;          /* fills emitted (F for a market that overflowed) */
    int64_t levels_emptied; /* price levels whose list became empty */
    int64_t overflows;      /* markets that ended with fill_counts = -1 */
} om_counters;

om_market *om_create(int32_t M, int32_t L, int32_t O, int32_t F, int32_t C);
om_market *om_clone(const om_market *src);
void om_destroy(om_market *mk);

/* AddTwoSidedQuotes (market.cu:458-535) followed by MatchAllMarkets
 * (market.cu:537-571). The 9 fill arrays are caller-owned, [M][F] (counts [M]).
 * nthreads > 1 runs markets in parallel with OpenMP (markets are independent).
 * counters may be NULL. */
void om_add_two_sided_quotes(om_market *mk, const int32_t *bid_px, const int32_t *bid_sz,
                             const int32_t *ask_px, const int32_t *ask_sz,
                             const int32_t *customer_ids, int32_t *fill_prices,
                             int32_t *fill_sizes, int32_t *fill_customer_ids,
                             int32_t *fill_quoter_ids, uint8_t *fill_is_sell_quote,
                             int32_t *fill_quote_sizes, int32_t *fill_tid,
                             int32_t *fill_quote_tid, int32_t *fill_counts, int nthreads,
                             om_counters *counters);

/* GetBBOs (market.cu:573-597, kernel :280-320). */
void om_get_bbos(const om_market *mk, int32_t *best_bid_prices, int32_t *best_bid_sizes,
                 int32_t *best_ask_prices, int32_t *best_ask_sizes, int nthreads);

/* BBOBatch::UpdateLastPrices (market.cu:798-825, kernel :767-786). */
void om_update_last_prices(int32_t *last_prices, const int32_t *fill_counts,
                           const int32_t *fill_prices, int32_t num_markets, int32_t max_fills);

void om_reset(om_market *mk);                                /* market.cu:693-716 */
void om_clear_quotes(om_market *mk, const uint8_t *reset);   /* market.cu:718-756 */

/* ToString (market.cu:599-691). Writes at most buflen bytes (NUL-terminated)
 * and returns the full length of the text. */
size_t om_to_string(const om_market *mk, int32_t market_id, char *buf, size_t buflen);

#ifdef __cplusplus
}
#endif
#endif
