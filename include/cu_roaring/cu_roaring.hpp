// Umbrella header -- counterpart of include/cu_roaring/cu_roaring.cuh.
#pragma once
#include "cu_roaring/types.hpp"
#include "cu_roaring/detail/utils.hpp"
#include "cu_roaring/detail/promote.hpp"
#include "cu_roaring/detail/upload.hpp"
#include "cu_roaring/detail/upload_ids.hpp"
#include "cu_roaring/detail/set_ops.hpp"
#include "cu_roaring/detail/decompress.hpp"
#include "cu_roaring/detail/to_csr.hpp"
#include "cu_roaring/detail/serialize.hpp"
#include "cu_roaring/detail/topk.hpp"
#include "cu_roaring/device/make_view.hpp"
