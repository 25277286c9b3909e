// CentroidMerge — merge every .centroid snapshot of a directory into k
// centers (reference: include/tensor/centroid/centroid_merge.hpp,
// src/centroid/centroid_merge.cpp:12-31).  Throws std::runtime_error when
// the directory holds no snapshot.
#pragma once
#include <string>

namespace tensor::centroid {

struct CentroidMerge {
    static void run(const std::string& snapshot_dir, const std::string& out_path, int k);
};

}  // namespace tensor::centroid
