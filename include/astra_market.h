/*
 * astra_market.h -- C ABI of the MI355X (gfx950) VecMarket order-matching engine.
 *
 * This is the drop-in boundary for the reference engine's C++ class
 * astra::order_matching::VecMarket (nlyu1/astra-cuda src/order_matching/market.h:121-350)
 * and its pybind module (src/pybind/order_matching/market_bindings.cc:14-73).
 * Every entry point takes plain device pointers, sizes and a HIP stream (as
 * void*, 0 = the null stream); nothing here allocates device memory. The book
 * state lives in a caller-provided workspace of astra_market_workspace_size()
 * bytes, so a PyTorch (or any other) host keeps ownership of all device memory.
 *
 * Return value of every int function: 0 on success, otherwise an error code
 * (ASTRA_ERR_*) with a message in astra_last_error() (per host thread). The
 * message text follows the reference's "Astra Fatal Error" convention
 * (src/utils/astra_utils.cc:13-18, astra_utils.h:116-131) minus the prefix.
 *
 * All kernels run on the stream passed in; calls are asynchronous except
 * astra_market_to_string (which synchronises the stream to read the book).
 */
#ifndef ASTRA_MARKET_H
#define ASTRA_MARKET_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference compile-time caps and sentinel, market.h:56-61. */
#define ASTRA_MAX_MARKETS (2048 * 2048)
#define ASTRA_PRICE_LEVELS 128
#define ASTRA_MAX_ACTIVE_ORDERS_PER_MARKET 1024
#define ASTRA_MAX_ACTIVE_FILLS_PER_MARKET 1024
#define ASTRA_NULL_INDEX (-1)
#define ASTRA_MAX_CUSTOMERS 1024

/* Caps accepted with ASTRA_FLAG_EXTENDED_SHAPES (a superset of the reference,
 * which rejects e.g. the deep-book shape L=512, O=F=4096 at market.cu:339-341). */
#define ASTRA_EXT_MAX_PRICE_LEVELS 1024
#define ASTRA_EXT_MAX_ORDERS 32768
#define ASTRA_EXT_MAX_FILLS 65536
#define ASTRA_EXT_MAX_CUSTOMERS 65536

#define ASTRA_FLAG_EXTENDED_SHAPES 1

#define ASTRA_OK 0
#define ASTRA_ERR_INVALID_ARGUMENT 1
#define ASTRA_ERR_HIP 2

typedef struct astra_market astra_market; /* opaque engine handle */

/* Message of the last failed call on this host thread ("" if none). */
const char *astra_last_error(void);

/* Device bytes the book state of this shape needs (validates the shape the
 * same way astra_market_create does). */
int astra_market_workspace_size(int32_t num_markets, int32_t max_price_levels,
                                int32_t max_active_orders_per_market,
                                int32_t max_active_fills_per_market, int32_t num_customers,
                                int32_t flags, size_t *bytes);

/* VecMarket::VecMarket (market.cu:326-383; market.h:138-140). Checks the caps
 * (market.cu:338-350) and the device id, then initialises the workspace on
 * `stream` to the empty book: all levels NULL, slot counters 0, portfolios 0,
 * the TID counter (a word of the workspace) 0. threads_per_block is validated
 * (0 < tpb <= 1024) but has no effect on results, as in the reference. */
int astra_market_create(int32_t num_markets, int32_t max_price_levels,
                        int32_t max_active_orders_per_market, int32_t max_active_fills_per_market,
                        int32_t num_customers, int device_id, int32_t threads_per_block,
                        int32_t flags, void *workspace, size_t workspace_bytes, void *stream,
                        astra_market **out);

/* VecMarket::~VecMarket (market.cu:413-418): synchronises the device, frees
 * the handle (not the workspace). */
int astra_market_destroy(astra_market *market);

/* VecMarket copy constructor (market.cu:385-411): copies the whole book
 * (device-to-device on `stream`), TID counter included, into dst_workspace. */
int astra_market_clone(const astra_market *src, void *dst_workspace, size_t dst_workspace_bytes,
                       void *stream, astra_market **out);

/* VecMarket::AddTwoSidedQuotes + MatchAllMarkets (market.cu:458-571).
 * Inputs: five int32 [M] device arrays. Outputs: the FillBatch (market.h:64-92),
 * eight [M,F] arrays (fill_is_sell_quote as one byte 0/1) and int32 [M]
 * fill_counts. Adds the bid then the ask of each market (TIDs base, base+1),
 * matches, and advances the TID counter by 2. The base is read from the
 * workspace by the kernel, not passed by the host: a launch captured in a HIP
 * graph replays with advancing TIDs (the reference passes it as an argument,
 * market.cu:520,531; see astra_market_get_tid). */
int astra_market_add_two_sided_quotes(astra_market *market, const int32_t *bid_px,
                                      const int32_t *bid_sz, const int32_t *ask_px,
                                      const int32_t *ask_sz, const int32_t *customer_ids,
                                      int32_t *fill_prices, int32_t *fill_sizes,
                                      int32_t *fill_customer_ids, int32_t *fill_quoter_ids,
                                      uint8_t *fill_is_sell_quote, int32_t *fill_quote_sizes,
                                      int32_t *fill_tid, int32_t *fill_quote_tid,
                                      int32_t *fill_counts, void *stream);

/* astra_market_add_two_sided_quotes with the fill rows in one int32 [M, F, 8]
 * array (16-byte aligned): row (m, k) = {price, size, taker, quoter, is_sell (0/1),
 * quote size, tid, quote tid}, the eight FillBatch fields of market.h:64-92 side by
 * side, so a row is one 32-byte write instead of eight scattered ones. No
 * counterpart in the reference: an alternative layout of the same FillBatch
 * (the Python layer exposes the eight fields as strided [M, F] views of it). */
int astra_market_add_two_sided_quotes_rows(astra_market *market, const int32_t *bid_px,
                                           const int32_t *bid_sz, const int32_t *ask_px,
                                           const int32_t *ask_sz, const int32_t *customer_ids,
                                           int32_t *fill_rows, int32_t *fill_counts,
                                           void *stream);

/* `steps` consecutive astra_market_add_two_sided_quotes calls in one launch.
 * No counterpart in the reference: a caller with the quotes of several steps
 * in hand (benchmarks, replays) runs them as one multi-step kernel in which each
 * wavefront goes on to its markets' next step without a grid-wide wait between
 * steps. The inputs are int32 [steps, M] arrays (row k = step k's quotes, TID
 * base = the counter + 2k); the state afterwards (book, portfolios, TID counter,
 * the fill batch, the BBO cache astra_market_get_bbos reads) is exactly that of
 * the `steps` single calls, so the fill batch holds the last step's fills
 * (rows beyond its count hold earlier steps' rows, as they would).
 * fill_rows non-NULL selects the [M, F, 8] row layout of
 * astra_market_add_two_sided_quotes_rows and the eight field pointers are not
 * used. step_fill_counts (int32 [steps, M]) receives every step's fill_counts and
 * step_bbos (int32 [4, steps, M]: best bid price, bid size, ask price, ask size)
 * every step's GetBBOs; either may be NULL. steps = 0 does nothing. */
int astra_market_add_two_sided_quotes_steps(
    astra_market *market, int32_t steps, const int32_t *bid_px, const int32_t *bid_sz,
    const int32_t *ask_px, const int32_t *ask_sz, const int32_t *customer_ids,
    int32_t *fill_prices, int32_t *fill_sizes, int32_t *fill_customer_ids,
    int32_t *fill_quoter_ids, uint8_t *fill_is_sell_quote, int32_t *fill_quote_sizes,
    int32_t *fill_tid, int32_t *fill_quote_tid, int32_t *fill_rows, int32_t *fill_counts,
    int32_t *step_fill_counts, int32_t *step_bbos, void *stream);

/* VecMarket::GetBBOs (market.cu:573-597): four int32 [M] outputs. The values
 * are those of the book as the last mutating call left it: the matching kernel
 * leaves the best levels' prices and head slots, and this call reads the head
 * orders' sizes from the book (get_bbo_kernel, market.cu:280-320, scans for the
 * same levels and reads the same sizes). */
int astra_market_get_bbos(const astra_market *market, int32_t *best_bid_prices,
                          int32_t *best_bid_sizes, int32_t *best_ask_prices,
                          int32_t *best_ask_sizes, void *stream);

/* BBOBatch::UpdateLastPrices (market.cu:798-825). */
int astra_update_last_prices(int32_t *last_prices, const int32_t *fill_counts,
                             const int32_t *fill_prices, int32_t num_markets,
                             int32_t max_fills, void *stream);

/* BBOBatch::UpdateLastPrices for a FillBatch in the row layout of
 * astra_market_add_two_sided_quotes_rows. */
int astra_update_last_prices_rows(int32_t *last_prices, const int32_t *fill_counts,
                                  const int32_t *fill_rows, int32_t num_markets,
                                  int32_t max_fills, void *stream);

/* Fill `count` int32 words with `value` on `stream` (used for FillBatch::Reset,
 * market.cu:758-760, and BBOBatch::Reset, market.cu:788-796). */
int astra_fill_i32(int32_t *dst, int64_t count, int32_t value, void *stream);

/* VecMarket::Reset (market.cu:693-716). */
int astra_market_reset(astra_market *market, void *stream);

/* VecMarket::ClearQuotes (market.cu:718-756): reset_mask is a byte [M] device
 * array (torch.bool); selected markets get an empty book and slot counter 0;
 * portfolios and the TID counter are kept. */
int astra_market_clear_quotes(astra_market *market, const uint8_t *reset_mask, void *stream);

/* VecMarket::GetCustomerPortfolios (market.h:294-296): device address of the
 * live int32 [M, C, 2] portfolio array inside the workspace. */
int astra_market_portfolios(const astra_market *market, int32_t **portfolios);

/* The shape the market was created with (num_markets_, max_price_levels_, ...,
 * market.h:320-330). Any pointer may be NULL. */
int astra_market_shape(const astra_market *market, int32_t *num_markets, int32_t *max_price_levels,
                       int32_t *max_active_orders_per_market, int32_t *max_active_fills_per_market,
                       int32_t *num_customers);

/* VecMarket::ToString (market.cu:599-691). Synchronises `stream`, formats the
 * book of market_id into buf (NUL-terminated, truncated to buflen) and stores
 * the full text length in *needed. */
int astra_market_to_string(const astra_market *market, int32_t market_id, char *buf,
                           size_t buflen, size_t *needed, void *stream);

/* Diagnostic, no counterpart in the reference: while `counters` (int64 [11],
 * device memory, caller-zeroed) is set, astra_market_add_two_sided_quotes also
 * adds to [0..10] the accepted order inserts, fill rows written (F for a market
 * that overflowed), price levels emptied, markets that overflowed, overflows
 * reached by fast-forwarding a repeating loop state, matching-loop passes,
 * markets finished from a staged (LDS) copy of their book, markets whose
 * book crossed (that entered the matching loop), runs of zero-size fill rows
 * listed on a staged book, the rows of those runs, and the best levels whose
 * head size the call left uncached (which astra_market_get_bbos then reads
 * from the book's order records).
 * These are the work counts of the algorithmic-byte roofline. NULL switches it
 * off (the default); the timed path never has it on. */
int astra_market_set_stats(astra_market *market, int64_t *counters);

/* The TID counter (market.h:338, the base TID of the next call). The reference
 * keeps it on the host and passes it to its kernels as an argument
 * (market.cu:520,531); here every market keeps a copy in the workspace, which
 * the matching kernel reads and advances with the market's other words, so that
 * calls captured in a HIP graph replay with advancing TIDs (every call steps
 * every market, so the copies agree). get: copies it to the host on `stream` and
 * synchronises the stream. set: writes every copy on `stream` (fill kernels, so
 * the call can be captured too). */
int astra_market_get_tid(const astra_market *market, int32_t *tid, void *stream);
int astra_market_set_tid(astra_market *market, int32_t tid, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ASTRA_MARKET_H */
