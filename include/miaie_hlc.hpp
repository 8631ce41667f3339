// miaie_hlc.hpp — launch targets of the `__kernel__` templates that
// aiehlc_amd/hlc.py writes into rewritten host sources.
//
// aiehlc turns each `__kernel__ NAME` into
//   template <int Col, int Row, int colstart, int rowstart, int M, int N, int K,
//             typename... Args> inline void NAME(Args&&... args)
// (src/llvm/aiehlc.cc:583-588), called as perf<1,1,4,4,256,16,64>(phy, phy_out)
// (example/nokernelload/aie_nokernelload.cc:130).  The rewritten template
// forwards to miaie_hlc::launch<KIND, Col, Row, colstart, rowstart, M, N, K>:
//   - two integer arguments are DDR addresses (XAie_MemGetDevAddr values):
//     the kernel runs on the Col x Row tiles from (colstart, rowstart) of the
//     aie-rt-shaped facade, reading its input window from the first address
//     and writing its output to the second (XAie_MiaieRunOnDdr);
//   - otherwise the arguments are device pointers (and scalars) for the miaie
//     launch templates of miaie.hpp, on the thread's current miaie::Context.
// Failures throw miaie::Error.
#ifndef MIAIE_HLC_HPP
#define MIAIE_HLC_HPP

#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>

#include "miaie.hpp"
#include "miaie_xaie.h"

namespace miaie_hlc {

enum class Kernel {
  perf_u8,   // uint8 MAC probe (aie_nokernelload.cc:50-83)
  mm,        // int32 window NT GEMM (aieml_mm.cc:41-93)
  perf,      // uint32 window NT GEMM (aieml_perf.cc:61-83)
  gemm_i8,   // int8 GEMM + requant (device pointers only)
  gemm_bf16  // bf16 GEMM (device pointers only)
};

template <Kernel KIND>
const XAie_MiaieKernel* descriptor() {
  if constexpr (KIND == Kernel::perf_u8) return &miaie_xaie_perf_u8;
  if constexpr (KIND == Kernel::mm) return &miaie_xaie_mm;
  if constexpr (KIND == Kernel::perf) return &miaie_xaie_perf;
  return nullptr;
}

template <typename... Args>
constexpr bool ddr_call() {
  if constexpr (sizeof...(Args) != 2)
    return false;
  else
    return (std::is_integral_v<std::decay_t<Args>> && ...);
}

template <Kernel KIND, int Col, int Row, int colstart, int rowstart, int M, int N, int K, typename... Args>
void launch(Args&&... args) {
  static_assert(Col >= 1 && Row >= 1 && colstart >= 0 && rowstart >= 0, "tile range");
  if constexpr (ddr_call<Args...>()) {
    static_assert(KIND == Kernel::perf_u8 || KIND == Kernel::mm || KIND == Kernel::perf,
                  "this kernel takes device pointers, not DDR addresses");
    static_assert(KIND == Kernel::perf_u8 || (M == 16 && N == 16 && K == 16),
                  "the tile window kernels mm / perf are 16 x 16 x 16");
    const uint64_t addr[2] = {static_cast<uint64_t>(args)...};
    const AieRC rc = XAie_MiaieRunOnDdr(descriptor<KIND>(), Col, Row, colstart, rowstart, addr[0], addr[1]);
    if (rc != XAIE_OK) throw miaie::Error(static_cast<int>(rc), XAie_MiaieLastError(nullptr));
  } else if constexpr (KIND == Kernel::perf_u8) {
    miaie::dot_probe<Col, Row, colstart, rowstart, M, N, K>(std::forward<Args>(args)...);
  } else if constexpr (KIND == Kernel::mm) {
    miaie::mm<Col, Row, colstart, rowstart, M, N, K>(std::forward<Args>(args)...);
  } else if constexpr (KIND == Kernel::perf) {
    miaie::perf<Col, Row, colstart, rowstart, M, N, K>(std::forward<Args>(args)...);
  } else if constexpr (KIND == Kernel::gemm_i8) {
    miaie::gemm_i8<Col, Row, colstart, rowstart, M, N, K>(std::forward<Args>(args)...);
  } else {
    miaie::gemm_bf16<Col, Row, colstart, rowstart, M, N, K>(std::forward<Args>(args)...);
  }
}

}  // namespace miaie_hlc

#endif  // MIAIE_HLC_HPP
