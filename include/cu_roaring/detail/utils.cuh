// Drop-in name of the reference header; see utils.hpp.
#pragma once
#include "cu_roaring/detail/utils.hpp"
