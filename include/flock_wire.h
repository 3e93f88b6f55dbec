/*
 * flock_wire.h -- the FLK1 activation frame (web/js/wire.mjs) for a worker
 * whose activations live on the GPU: the f16 payload conversion runs on the
 * device, the 20-byte header is packed and checked on the host.
 *
 * Frame: "FLK1" (u32 0x314b4c46, little-endian) | seq u32 | hidden u32 |
 * offset u32 | flags u32 | n f16 values (wire.mjs:7-16). flags bit 0 = reset,
 * bit 1 = replay (wire.mjs:63-64).
 */
#ifndef FLOCK_WIRE_H
#define FLOCK_WIRE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLK_WIRE_MAGIC 0x314b4c46u
#define FLK_WIRE_HEADER_BYTES 20u
#define FLK_WIRE_RESET 1u
#define FLK_WIRE_REPLAY 2u

/* f32 -> f16 bits, round to nearest even, subnormals, overflow to inf, NaN to
 * sign | 0x7e00: f32to16 (wire.mjs:33-53) on n DEVICE values. */
int32_t flk_f32_to_f16(const float* in, uint16_t* out, uint64_t n);

/* f16 bits -> f32: f16to32 (wire.mjs:55-61), inf kept, NaN to the quiet NaN
 * 0x7fc00000, on n DEVICE values. */
int32_t flk_f16_to_f32(const uint16_t* in, float* out, uint64_t n);

/* The header of pack (wire.mjs:66-78) into 20 HOST bytes. */
int32_t flk_wire_header_pack(uint32_t seq, uint32_t hidden, uint32_t offset, uint32_t flags,
                             void* out20);

/* The header checks of unpack (wire.mjs:80-88) on a HOST frame of frame_bytes:
 * FLK_ERR_ARG "not a flock frame" if the magic is wrong or the frame is
 * shorter than the header; writes the fields and the payload's value count. */
int32_t flk_wire_header_unpack(const void* frame, uint64_t frame_bytes, uint32_t* seq,
                               uint32_t* hidden, uint32_t* offset, uint32_t* flags,
                               uint64_t* n_values);

#ifdef __cplusplus
}
#endif

#endif /* FLOCK_WIRE_H */
