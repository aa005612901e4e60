// nnz-balanced contiguous row partition (reference: spmm_multigpu.cu:26-40).

#include "spmm/partition.h"

#include <algorithm>
#include <stdexcept>

namespace spmm {

std::vector<int> nnz_balanced_bounds(const CSR& h_A, int parts) {
    if (parts < 1) throw std::runtime_error("nnz_balanced_bounds: parts must be >= 1");
    std::vector<int> bounds(static_cast<size_t>(parts) + 1, 0);
    bounds[parts] = h_A.num_rows;
    const long long total = h_A.nnz;
    int r = 0;
    for (int g = 1; g < parts; ++g) {
        const long long target = total * g / parts;
        // rows are visited once over the whole loop: targets only grow
        while (r < h_A.num_rows && h_A.row_ptr[r] < target) ++r;
        bounds[g] = r;
    }
    for (int g = 1; g <= parts; ++g) bounds[g] = std::max(bounds[g], bounds[g - 1]);
    return bounds;
}

std::vector<int> nnz_split_rows(const CSR& h_A, int parts) {
    if (parts < 1) throw std::runtime_error("nnz_split_rows: parts must be >= 1");
    if (h_A.nnz < 1 || h_A.num_rows < 1) {
        throw std::runtime_error("nnz_split_rows: needs at least one nonzero");
    }
    std::vector<int> rows(static_cast<size_t>(parts) + 1, 0);
    rows[parts] = h_A.num_rows;
    const long long total = h_A.nnz;
    const int* rp = h_A.row_ptr;
    for (int g = 1; g < parts; ++g) {
        const long long p = total * g / parts;
        // last r in [0, num_rows) with row_ptr[r] <= p
        const int* it = std::upper_bound(rp, rp + h_A.num_rows, static_cast<int>(p));
        rows[g] = static_cast<int>(it - rp) - 1;
    }
    return rows;
}

}  // namespace spmm
