// Drop-in name of the reference header; see upload_ids.hpp.
#pragma once
#include "cu_roaring/detail/upload_ids.hpp"
