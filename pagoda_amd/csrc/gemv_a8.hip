// gemv_a8.hip — A8 instantiations of the GEMV templates in gemv_impl.h.
#include "gemv_impl.h"

namespace pgd {
namespace gemv {

void run_a8(const GemvArgs& a, int nrows, int x_f16, int epi, hipStream_t s) {
  if (epi == EPI_SWIGLU) {
    launch_rows<A8, false, EPI_SWIGLU>(a, nrows, s);
  } else if (x_f16) {
    if (epi == EPI_RES) launch_rows<A8, true, EPI_RES>(a, nrows, s);
    else launch_rows<A8, true, EPI_STORE>(a, nrows, s);
  } else {
    if (epi == EPI_RES) launch_rows<A8, false, EPI_RES>(a, nrows, s);
    else launch_rows<A8, false, EPI_STORE>(a, nrows, s);
  }
}

}  // namespace gemv
}  // namespace pgd
