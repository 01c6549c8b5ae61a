// Drop-in name of the reference header; see set_ops.hpp.
#pragma once
#include "cu_roaring/detail/set_ops.hpp"
