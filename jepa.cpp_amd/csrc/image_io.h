// image_io.h - image file decoders behind jepa_load_image_rgb (image_io.cpp, jpeg_decode.cpp).
#pragma once
#include <cstddef>
#include <cstdint>

// Baseline JPEG in memory -> malloc'd RGB8 HWC (free with jepa_free); nullptr and a logged reason
// (naming `path`) on failure.
uint8_t * decode_jpeg(const uint8_t * data, size_t n, int * h, int * w, const char * path);
