// Hand-written fused attention template for gfx950.
#pragma once
