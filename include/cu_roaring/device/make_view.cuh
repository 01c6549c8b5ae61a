// Drop-in name of the reference header; see make_view.hpp.
#pragma once
#include "cu_roaring/device/make_view.hpp"
