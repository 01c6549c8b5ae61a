// Drop-in name of the reference header; see promote.hpp.
#pragma once
#include "cu_roaring/detail/promote.hpp"
