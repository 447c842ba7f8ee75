// Handle types behind the flat C APIs (tinymlp_capi.h, nerf_capi.h).
#pragma once

#include "TinyMLP.h"
#include "TinyMLPHashGrid.h"
#include "tinymlp_capi.h"

struct TmlpGrid {
    TinyMLPHashGrid* g;
    bool owned = true;  // false for a view into an InstantNerf's density head
};

struct TmlpNet {
    TinyMLP* n;
    bool owned = true;  // false for a view into an InstantNerf's color head
};
