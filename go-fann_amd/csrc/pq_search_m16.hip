// pq_search_m16.hip -- PQ traversal kernels for pq_dim = 16 (instantiated here
// so the kernel variants compile in parallel).
#include "traversal.hpp"

namespace gofann {
template int pq_search_m<16>(GOFANN_PQ_SEARCH_M_ARGS);

}  // namespace gofann
