// Drop-in name of the reference header; see upload.hpp.
#pragma once
#include "cu_roaring/detail/upload.hpp"
