// Drop-in name of the reference header; see cu_roaring.hpp.
#pragma once
#include "cu_roaring/cu_roaring.hpp"
