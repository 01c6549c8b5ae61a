// Drop-in name of the reference header; see roaring_wavefront_query.hpp.
#pragma once
#include "cu_roaring/device/roaring_wavefront_query.hpp"
