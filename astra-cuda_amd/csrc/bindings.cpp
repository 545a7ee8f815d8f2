// bindings.cpp -- the compiled Python binding of the engine: module astra_cuda._C
// with the submodule order_matching, class for class the reference's pybind
// module (nlyu1/astra-cuda src/pybind/order_matching/market_bindings.cc:14-73,
// src/pybind/bindings.cc:16-24) over the C ABI of include/astra_market.h.
//
// Validation runs here in C++ with the reference's checks and messages
// (market.cu:338-350 for the constructor, :467-505 for AddTwoSidedQuotes);
// a failed check prints "Astra Fatal Error: ..." to stderr and raises
// RuntimeError, as AstraFatalError does (src/utils/astra_utils.cc:13-18).
// Every call runs on PyTorch's current HIP stream of the market's device. The
// book lives in a workspace tensor the market owns; FillBatch and BBOBatch hold
// their tensors as plain fields (def_readwrite, as in the reference).
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <cstdio>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "astra_market.h"

namespace py = pybind11;

namespace astra_bind {

[[noreturn]] void fatal(const std::string &msg) {
  std::fprintf(stderr, "Astra Fatal Error: %s\n\n", msg.c_str());
  std::fflush(stderr);
  throw std::runtime_error("Astra Fatal Error: " + msg);
}

void check(int rc) {
  if (rc != ASTRA_OK) fatal(astra_last_error());
}

// ASTRA_CHECK_EQ's text (src/utils/astra_utils.h:116-131), this file's name in
// place of market.cu.
#define BIND_CHECK_EQ(x_exp, y_exp)                                                             \
  do {                                                                                          \
    const long long x_ = (long long)(x_exp), y_ = (long long)(y_exp);                           \
    if (x_ != y_)                                                                               \
      fatal(std::string("bindings.cpp:") + std::to_string(__LINE__) + " " #x_exp " == " #y_exp \
            "\n" #x_exp " = " + std::to_string(x_) + ", " #y_exp " = " + std::to_string(y_));   \
  } while (false)

void *stream_of(int device) {
  return reinterpret_cast<void *>(c10::hip::getCurrentHIPStream((c10::DeviceIndex)device).stream());
}

// FillBatch (market.h:64-92).
struct FillBatch {
  torch::Tensor fill_prices, fill_sizes, fill_customer_ids, fill_quoter_ids, fill_is_sell_quote,
      fill_quote_sizes, fill_tid, fill_quote_tid, fill_counts;

  // FillBatch::Reset (market.cu:758-760).
  void Reset() {
    check(astra_fill_i32(fill_counts.data_ptr<int32_t>(), fill_counts.numel(), 0,
                         stream_of(fill_counts.get_device())));
  }
};

// BBOBatch (market.h:95-119).
struct BBOBatch {
  torch::Tensor best_bid_prices, best_bid_sizes, best_ask_prices, best_ask_sizes, last_prices;

  // BBOBatch::Reset (market.cu:788-796).
  void Reset() {
    for (torch::Tensor *t : {&best_bid_prices, &best_bid_sizes, &best_ask_prices, &best_ask_sizes,
                             &last_prices})
      check(astra_fill_i32(t->data_ptr<int32_t>(), t->numel(), 0, stream_of(t->get_device())));
  }

  // BBOBatch::UpdateLastPrices (market.cu:798-825).
  void UpdateLastPrices(const FillBatch &fills) {
    const torch::Tensor &fc = fills.fill_counts, &fp = fills.fill_prices;
    if (fc.device() != last_prices.device())
      fatal("fills.fill_counts.device() == last_prices.device()");
    if (fp.device() != last_prices.device())
      fatal("fills.fill_prices.device() == last_prices.device()");
    const int64_t M = fc.size(0), F = fp.size(1);
    BIND_CHECK_EQ(last_prices.size(0), M);
    BIND_CHECK_EQ(fp.size(0), M);
    for (const torch::Tensor *t : std::initializer_list<const torch::Tensor *>{&last_prices, &fc, &fp})
      if (t->scalar_type() != torch::kInt32 || !t->is_contiguous())
        fatal("UpdateLastPrices needs contiguous int32 tensors");
    check(astra_update_last_prices(last_prices.data_ptr<int32_t>(), fc.data_ptr<int32_t>(),
                                   fp.data_ptr<int32_t>(), (int32_t)M, (int32_t)F,
                                   stream_of(last_prices.get_device())));
  }
};

// VecMarket (market.h:121-350).
class VecMarket {
 public:
  // VecMarket::VecMarket (market.cu:326-383).
  VecMarket(int32_t num_markets, int32_t max_price_levels, int32_t max_active_orders_per_market,
            int32_t max_active_fills_per_market, int32_t num_customers, int device_id,
            int32_t threads_per_block)
      : M_(num_markets), L_(max_price_levels), O_(max_active_orders_per_market),
        F_(max_active_fills_per_market), C_(num_customers), device_(device_id),
        tpb_(threads_per_block) {
    size_t bytes = 0;
    check(astra_market_workspace_size(M_, L_, O_, F_, C_, 0, &bytes));
    const int64_t ndev = (int64_t)torch::cuda::device_count();
    if (device_ < 0 || device_ >= ndev)  // market.cu:349-350
      fatal("bindings.cpp device_id < device_count\ndevice_id = " + std::to_string(device_) +
            ", device_count = " + std::to_string(ndev));
    allocate(bytes);
    astra_market *h = nullptr;
    check(astra_market_create(M_, L_, O_, F_, C_, device_, tpb_, 0, ws_.data_ptr(),
                              (size_t)ws_.numel(), stream_of(device_), &h));
    h_ = h;
    view_portfolios();
  }

  // The copy constructor (market.cu:385-411): a deep copy, TID counter included.
  VecMarket(const VecMarket &o)
      : M_(o.M_), L_(o.L_), O_(o.O_), F_(o.F_), C_(o.C_), device_(o.device_), tpb_(o.tpb_) {
    allocate((size_t)o.ws_.numel());
    astra_market *h = nullptr;
    check(astra_market_clone(o.h_, ws_.data_ptr(), (size_t)ws_.numel(), stream_of(device_), &h));
    h_ = h;
    view_portfolios();
  }

  VecMarket &operator=(const VecMarket &) = delete;

  // market.cu:413-418: synchronises the device.
  ~VecMarket() {
    if (h_) astra_market_destroy(h_);
  }

  // NewFillBatch (market.cu:420-439): zero-initialised tensors.
  FillBatch NewFillBatch() const {
    const auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(torch::kCUDA, device_);
    FillBatch b;
    b.fill_prices = torch::zeros({M_, F_}, i32);
    b.fill_sizes = torch::zeros({M_, F_}, i32);
    b.fill_customer_ids = torch::zeros({M_, F_}, i32);
    b.fill_quoter_ids = torch::zeros({M_, F_}, i32);
    b.fill_is_sell_quote = torch::zeros({M_, F_}, i32.dtype(torch::kBool));
    b.fill_quote_sizes = torch::zeros({M_, F_}, i32);
    b.fill_tid = torch::zeros({M_, F_}, i32);
    b.fill_quote_tid = torch::zeros({M_, F_}, i32);
    b.fill_counts = torch::zeros({M_}, i32);
    return b;
  }

  // NewBBOBatch (market.cu:441-456): all five tensors zero.
  BBOBatch NewBBOBatch() const {
    const auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(torch::kCUDA, device_);
    BBOBatch b;
    b.best_bid_prices = torch::zeros({M_}, i32);
    b.best_bid_sizes = torch::zeros({M_}, i32);
    b.best_ask_prices = torch::zeros({M_}, i32);
    b.best_ask_sizes = torch::zeros({M_}, i32);
    b.last_prices = torch::zeros({M_}, i32);
    return b;
  }

  // AddTwoSidedQuotes + MatchAllMarkets (market.cu:458-571).
  void AddTwoSidedQuotes(const torch::Tensor &bid_px, const torch::Tensor &bid_sz,
                         const torch::Tensor &ask_px, const torch::Tensor &ask_sz,
                         const torch::Tensor &customer_ids, FillBatch &fills) {
    const int64_t num_markets_ = M_;  // (the name the reference's messages show)
    BIND_CHECK_EQ(bid_px.size(0), num_markets_);  // market.cu:467-471
    BIND_CHECK_EQ(bid_sz.size(0), num_markets_);
    BIND_CHECK_EQ(ask_px.size(0), num_markets_);
    BIND_CHECK_EQ(ask_sz.size(0), num_markets_);
    BIND_CHECK_EQ(customer_ids.size(0), num_markets_);
    check_input(bid_px, "bid_px");  // market.cu:474-504
    check_input(bid_sz, "bid_sz");
    check_input(ask_px, "ask_px");
    check_input(ask_sz, "ask_sz");
    check_input(customer_ids, "customer_ids");
    check_fill(fills.fill_prices, "fill_prices", torch::kInt32, true);
    check_fill(fills.fill_sizes, "fill_sizes", torch::kInt32, true);
    check_fill(fills.fill_customer_ids, "fill_customer_ids", torch::kInt32, true);
    check_fill(fills.fill_quoter_ids, "fill_quoter_ids", torch::kInt32, true);
    check_fill(fills.fill_is_sell_quote, "fill_is_sell_quote", torch::kBool, true);
    check_fill(fills.fill_quote_sizes, "fill_quote_sizes", torch::kInt32, true);
    check_fill(fills.fill_tid, "fill_tid", torch::kInt32, true);
    check_fill(fills.fill_quote_tid, "fill_quote_tid", torch::kInt32, true);
    check_fill(fills.fill_counts, "fill_counts", torch::kInt32, false);
    check(astra_market_add_two_sided_quotes(
        h_, bid_px.data_ptr<int32_t>(), bid_sz.data_ptr<int32_t>(), ask_px.data_ptr<int32_t>(),
        ask_sz.data_ptr<int32_t>(), customer_ids.data_ptr<int32_t>(),
        fills.fill_prices.data_ptr<int32_t>(), fills.fill_sizes.data_ptr<int32_t>(),
        fills.fill_customer_ids.data_ptr<int32_t>(), fills.fill_quoter_ids.data_ptr<int32_t>(),
        reinterpret_cast<uint8_t *>(fills.fill_is_sell_quote.data_ptr<bool>()),
        fills.fill_quote_sizes.data_ptr<int32_t>(), fills.fill_tid.data_ptr<int32_t>(),
        fills.fill_quote_tid.data_ptr<int32_t>(), fills.fill_counts.data_ptr<int32_t>(),
        stream_of(device_)));
  }

  // GetBBOs (market.cu:573-597).
  void GetBBOs(BBOBatch &bbos) {
    for (auto [t, name] : {std::pair<torch::Tensor *, const char *>{&bbos.best_bid_prices, "best_bid_prices"},
                           {&bbos.best_bid_sizes, "best_bid_sizes"},
                           {&bbos.best_ask_prices, "best_ask_prices"},
                           {&bbos.best_ask_sizes, "best_ask_sizes"}}) {
      if (t->dim() != 1 || t->size(0) != M_ || t->scalar_type() != torch::kInt32)
        fatal(std::string("bbos.") + name + " must be an int32 tensor of shape [" +
              std::to_string(M_) + "]");
      if (!on_device(*t))
        fatal(std::string("bbos.") + name + " tensor must be on device " + std::to_string(device_));
      if (!t->is_contiguous()) fatal(std::string("bbos.") + name + " tensor must be contiguous");
    }
    check(astra_market_get_bbos(h_, bbos.best_bid_prices.data_ptr<int32_t>(),
                                bbos.best_bid_sizes.data_ptr<int32_t>(),
                                bbos.best_ask_prices.data_ptr<int32_t>(),
                                bbos.best_ask_sizes.data_ptr<int32_t>(), stream_of(device_)));
  }

  // ToString (market.cu:599-691); synchronises the current stream.
  std::string ToString(int32_t market_id) const {
    size_t need = 0;
    std::vector<char> buf(1 << 16);
    check(astra_market_to_string(h_, market_id, buf.data(), buf.size(), &need, stream_of(device_)));
    if (need >= buf.size()) {
      buf.resize(need + 1);
      check(astra_market_to_string(h_, market_id, buf.data(), buf.size(), &need, stream_of(device_)));
    }
    return std::string(buf.data(), need);
  }

  // GetCustomerPortfolios (market.h:294-296): the live [M, C, 2] tensor.
  torch::Tensor GetCustomerPortfolios() const { return portfolios_; }

  // CopyCustomerPortfoliosTo (market.h:285-292).
  void CopyCustomerPortfoliosTo(torch::Tensor buffer) const {
    BIND_CHECK_EQ(buffer.dim(), 3);
    BIND_CHECK_EQ(buffer.size(0), M_);
    BIND_CHECK_EQ(buffer.size(1), C_);
    BIND_CHECK_EQ(buffer.size(2), 2);
    buffer.copy_(portfolios_, /*non_blocking=*/false);
  }

  // Reset (market.cu:693-716).
  void Reset() { check(astra_market_reset(h_, stream_of(device_))); }

  // ClearQuotes (market.cu:718-756).
  void ClearQuotes(const torch::Tensor &reset_indices) {
    const int64_t num_markets_ = M_;
    BIND_CHECK_EQ(reset_indices.dim(), 1);
    BIND_CHECK_EQ(reset_indices.size(0), num_markets_);
    if (reset_indices.scalar_type() != torch::kBool)
      fatal("bindings.cpp reset_indices.dtype() == torch::kBool");
    if (!on_device(reset_indices))
      fatal("reset_indices tensor must be on device " + std::to_string(device_));
    const torch::Tensor r = reset_indices.contiguous();
    check(astra_market_clear_quotes(h_, reinterpret_cast<const uint8_t *>(r.data_ptr<bool>()),
                                    stream_of(device_)));
  }

  // The TID counter (market.h:338); reading it synchronises the current stream.
  int32_t GlobalTid() const {
    int32_t tid = 0;
    check(astra_market_get_tid(h_, &tid, stream_of(device_)));
    return tid;
  }

  int32_t num_markets() const { return M_; }

  // The workspace tensor (the book in the layout of include/astra_market.h), for
  // tools that copy a book between this binding and astra_cuda.order_matching.
  torch::Tensor Workspace() const { return ws_; }

 private:
  void allocate(size_t bytes) {
    ws_ = torch::empty({(int64_t)std::max<size_t>(bytes, 256)},
                       torch::TensorOptions().dtype(torch::kUInt8).device(torch::kCUDA, device_));
  }

  void view_portfolios() {
    int32_t *p = nullptr;
    check(astra_market_portfolios(h_, &p));
    const int64_t off = reinterpret_cast<uint8_t *>(p) - ws_.data_ptr<uint8_t>();
    portfolios_ = ws_.narrow(0, off, (int64_t)M_ * C_ * 8).view(torch::kInt32).view({M_, C_, 2});
  }

  bool on_device(const torch::Tensor &t) const {
    return t.is_cuda() && t.get_device() == device_;
  }

  void check_input(const torch::Tensor &t, const char *name) const {
    if (!on_device(t)) fatal(std::string(name) + " tensor must be on device " + std::to_string(device_));
    if (!t.is_contiguous()) fatal(std::string(name) + " tensor must be contiguous");
    if (t.scalar_type() != torch::kInt32)
      fatal(std::string(name) + " tensor must be int32, got " + std::string(c10::toString(t.scalar_type())));
  }

  void check_fill(const torch::Tensor &t, const char *name, c10::ScalarType dt, bool rows) const {
    if (!t.defined()) fatal(std::string("fills.") + name + " is not a tensor");
    const bool shape_ok = rows ? (t.dim() == 2 && t.size(0) == M_ && t.size(1) == F_)
                               : (t.dim() == 1 && t.size(0) == M_);
    if (!shape_ok || t.scalar_type() != dt)
      fatal(std::string("fills.") + name + " must be " + c10::toString(dt) + " of shape [" +
            std::to_string(M_) + (rows ? ", " + std::to_string(F_) : std::string()) + "]");
    if (!on_device(t)) fatal(std::string("fills.") + name + " tensor must be on device " + std::to_string(device_));
    if (!t.is_contiguous()) fatal(std::string("fills.") + name + " tensor must be contiguous");
  }

  int32_t M_, L_, O_, F_, C_;
  int device_;
  int32_t tpb_;
  astra_market *h_ = nullptr;
  torch::Tensor ws_, portfolios_;
};

}  // namespace astra_bind

// market_bindings.cc:14-73 and bindings.cc:16-24: the same submodule, classes,
// fields, methods, keyword names and constants; plus the C++-only surface the
// reference's game uses (Reset, ClearQuotes, CopyCustomerPortfoliosTo, the copy
// constructor, FillBatch::Reset, BBOBatch::Reset / UpdateLastPrices).
PYBIND11_MODULE(_C, m) {
  using namespace astra_bind;
  m.doc() = "astra_cuda compiled binding (MI355X engine)";
  py::module_ om = m.def_submodule("order_matching", "Order matching engine");
  py::class_<BBOBatch>(om, "BBOBatch")
      .def_readwrite("best_bid_prices", &BBOBatch::best_bid_prices)
      .def_readwrite("best_bid_sizes", &BBOBatch::best_bid_sizes)
      .def_readwrite("best_ask_prices", &BBOBatch::best_ask_prices)
      .def_readwrite("best_ask_sizes", &BBOBatch::best_ask_sizes)
      .def_readwrite("last_prices", &BBOBatch::last_prices)
      .def("reset", &BBOBatch::Reset)
      .def("update_last_prices", &BBOBatch::UpdateLastPrices, py::arg("fills"));
  py::class_<FillBatch>(om, "FillBatch")
      .def_readwrite("fill_prices", &FillBatch::fill_prices)
      .def_readwrite("fill_sizes", &FillBatch::fill_sizes)
      .def_readwrite("fill_customer_ids", &FillBatch::fill_customer_ids)
      .def_readwrite("fill_quoter_ids", &FillBatch::fill_quoter_ids)
      .def_readwrite("fill_is_sell_quote", &FillBatch::fill_is_sell_quote)
      .def_readwrite("fill_quote_sizes", &FillBatch::fill_quote_sizes)
      .def_readwrite("fill_tid", &FillBatch::fill_tid)
      .def_readwrite("fill_quote_tid", &FillBatch::fill_quote_tid)
      .def_readwrite("fill_counts", &FillBatch::fill_counts)
      .def("reset", &FillBatch::Reset);
  py::class_<VecMarket>(om, "VecMarket")
      .def(py::init<int32_t, int32_t, int32_t, int32_t, int32_t, int, int32_t>(),
           py::arg("num_markets"), py::arg("max_price_levels"),
           py::arg("max_active_orders_per_market"), py::arg("max_active_fills_per_market"),
           py::arg("num_customers") = 16, py::arg("device_id") = 0,
           py::arg("threads_per_block") = 64)
      .def("new_fill_batch", &VecMarket::NewFillBatch,
           "Create a new FillBatch with properly allocated tensors")
      .def("new_bbo_batch", &VecMarket::NewBBOBatch,
           "Create a new BBOBatch with properly allocated tensors")
      .def("add_two_sided_quotes", &VecMarket::AddTwoSidedQuotes, py::arg("bid_px"),
           py::arg("bid_sz"), py::arg("ask_px"), py::arg("ask_sz"), py::arg("customer_ids"),
           py::arg("fills"), "Add two-sided quotes (bid and ask) for all markets in parallel")
      .def("get_bbos", &VecMarket::GetBBOs, py::arg("bbos"),
           "Populate the best bid and offer (BBO) for all markets")
      .def("to_string", &VecMarket::ToString, py::arg("market_id"),
           "Return a string representation of a specific market's order book")
      .def("get_customer_portfolios", &VecMarket::GetCustomerPortfolios,
           py::return_value_policy::reference_internal, "Return a live view of customer portfolios")
      .def("copy_customer_portfolios_to", &VecMarket::CopyCustomerPortfoliosTo, py::arg("buffer"))
      .def("reset", &VecMarket::Reset)
      .def("clear_quotes", &VecMarket::ClearQuotes, py::arg("reset_indices"))
      .def("clone", [](const VecMarket &v) { return std::make_unique<VecMarket>(v); })
      .def("__copy__", [](const VecMarket &v) { return std::make_unique<VecMarket>(v); })
      .def("__deepcopy__", [](const VecMarket &v, py::dict) { return std::make_unique<VecMarket>(v); })
      .def_property_readonly("global_tid", &VecMarket::GlobalTid)
      .def_property_readonly("num_markets", &VecMarket::num_markets)
      .def_property_readonly("_workspace", &VecMarket::Workspace);
  om.attr("MAX_MARKETS") = ASTRA_MAX_MARKETS;
  om.attr("PRICE_LEVELS") = ASTRA_PRICE_LEVELS;
  om.attr("MAX_ACTIVE_ORDERS_PER_MARKET") = ASTRA_MAX_ACTIVE_ORDERS_PER_MARKET;
  om.attr("MAX_ACTIVE_FILLS_PER_MARKET") = ASTRA_MAX_ACTIVE_FILLS_PER_MARKET;
  om.attr("NULL_INDEX") = ASTRA_NULL_INDEX;
  om.attr("MAX_CUSTOMERS") = ASTRA_MAX_CUSTOMERS;
}
