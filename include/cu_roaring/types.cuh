// Drop-in name of the reference header; see types.hpp.
#pragma once
#include "cu_roaring/types.hpp"
