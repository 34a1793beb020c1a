// gemv_q50.hip — Q8_0 and Q5_0 instantiations of the GEMV templates in
// gemv_impl.h (GGML 32-weight blocks: the fallback types of Q4_K_M files for
// rows that are not whole 256-weight super-blocks).
#include "gemv_impl.h"

namespace pgd {
namespace gemv {

namespace {
template <class F>
void run_blocks(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) {
    launch_rows<F, false, EPI_SWIGLU>(a, nrows, s);
  } else if (x_f16) {
    if (epi == EPI_RES) launch_rows<F, true, EPI_RES>(a, nrows, s);
    else launch_rows<F, true, EPI_STORE>(a, nrows, s);
  } else {
    if (epi == EPI_RES) launch_rows<F, false, EPI_RES>(a, nrows, s);
    else launch_rows<F, false, EPI_STORE>(a, nrows, s);
  }
}
}  // namespace

void run_q80(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) { run_blocks<Q80>(a, nrows, x_f16, epi, s); }
void run_q50(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) { run_blocks<Q50>(a, nrows, x_f16, epi, s); }

}  // namespace gemv
}  // namespace pgd
