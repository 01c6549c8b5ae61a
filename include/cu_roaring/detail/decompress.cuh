// Drop-in name of the reference header; see decompress.hpp.
#pragma once
#include "cu_roaring/detail/decompress.hpp"
