// Drop-in name of the reference header; see types.hpp.
#pragma once
#include "cu_roaring_v2/types.hpp"
