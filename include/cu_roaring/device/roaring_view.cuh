// Drop-in name of the reference header; see roaring_view.hpp.
#pragma once
#include "cu_roaring/device/roaring_view.hpp"
