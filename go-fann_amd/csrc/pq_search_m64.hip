// pq_search_m64.hip -- PQ traversal kernels for pq_dim = 64 (instantiated here
// so the kernel variants compile in parallel).
#include "traversal.hpp"

namespace gofann {
template int pq_search_m<64>(GOFANN_PQ_SEARCH_M_ARGS);

}  // namespace gofann
