"""Byte layouts of the per-tile records (numpy codec).

A record holds one 64-key tile of one KV head.  Sizes are the reference's
(K8 8 KiB, K4 4 KiB, V16 16 KiB, V8 8 KiB, V4 4 KiB; decode.py:7-8); the byte
order inside a record is this implementation's, chosen so that each 1 KiB
fragment is one 32x32 MFMA operand (triattention_amd/csrc/common.h).  These
functions convert between records and logical [64 keys, 128] code arrays; they
are used by tests and by anything that persists or inspects caches, never by
the compute path.
"""
from __future__ import annotations

import numpy as np

BN, D = 64, 128


def _k8_index():
    o = np.arange(8192)
    F, L, j = o // 1024, (o // 16) % 64, o % 16
    kb, ks = F // 4, F % 4
    return kb * 32 + L % 32, ks * 32 + 16 * (L // 32) + j


def _v8_index():
    o = np.arange(8192)
    F, L, p = o // 1024, (o // 16) % 64, o % 16
    cb, kb = F // 2, F % 2
    return kb * 32 + 8 * (p // 4) + 4 * (L // 32) + p % 4, cb * 32 + L % 32


def _v16_index():
    o = np.arange(8192)  # fp16 element index
    F, L, e = o // 512, (o // 8) % 64, o % 8
    kh, kb, cb = F % 2, (F // 2) % 2, F // 4
    return kb * 32 + 8 * (2 * kh + e // 4) + 4 * (L // 32) + e % 4, cb * 32 + L % 32


def _nibble_index():
    """For each byte of a 4-bit record: the 8-bit-layout byte of its low and high nibble.

    Fragment F's 8-byte word pair of lane L sits at byte (F // 2) * 1024 + 16 L + 8 (F % 2),
    so one 16-byte access per lane fetches two fragments."""
    o = np.arange(4096)
    F = 2 * (o // 1024) + (o % 16) // 8
    L, bb = (o // 16) % 64, o % 8
    base = F * 1024 + L * 16
    lo = np.where(bb < 4, bb, 8 + (bb - 4))
    return base + lo, base + lo + 4


K8_KEY, K8_FEAT = _k8_index()
V8_KEY, V8_CH = _v8_index()
V16_KEY, V16_CH = _v16_index()
NIB_LO, NIB_HI = _nibble_index()


def _bytes(rec, size):
    a = np.ascontiguousarray(rec).view(np.uint8)
    return a.reshape(-1, size)


def unpack_k8(rec):
    """K8 records -> int8 codes [N, 64, 128] (key, feature)."""
    r = _bytes(rec, 8192).view(np.int8)
    out = np.empty((r.shape[0], BN, D), np.int8)
    out[:, K8_KEY, K8_FEAT] = r
    return out


def pack_k8(codes):
    c = np.asarray(codes, np.int8).reshape(-1, BN, D)
    return np.ascontiguousarray(c[:, K8_KEY, K8_FEAT]).view(np.uint8)


def _unpack4(rec, key, other):
    r = _bytes(rec, 4096)
    flat = np.empty((r.shape[0], 8192), np.int8)
    lo, hi = (r & 15).astype(np.int8), (r >> 4).astype(np.int8)
    flat[:, NIB_LO] = np.where(lo > 7, lo - 16, lo)
    flat[:, NIB_HI] = np.where(hi > 7, hi - 16, hi)
    out = np.empty((r.shape[0], BN, D), np.int8)
    out[:, key, other] = flat
    return out


def _pack4(codes, key, other):
    c = np.asarray(codes, np.int8).reshape(-1, BN, D)
    flat = (c[:, key, other].astype(np.int16) & 15).astype(np.uint8)
    return np.ascontiguousarray(flat[:, NIB_LO] | (flat[:, NIB_HI] << 4))


def unpack_k4(rec):
    """K4 records -> signed 4-bit codes [N, 64, 128]."""
    return _unpack4(rec, K8_KEY, K8_FEAT)


def pack_k4(codes):
    return _pack4(codes, K8_KEY, K8_FEAT)


def unpack_v8(rec):
    """V8 records -> int8 codes [N, 64 keys, 128 channels]."""
    r = _bytes(rec, 8192).view(np.int8)
    out = np.empty((r.shape[0], BN, D), np.int8)
    out[:, V8_KEY, V8_CH] = r
    return out


def pack_v8(codes):
    c = np.asarray(codes, np.int8).reshape(-1, BN, D)
    return np.ascontiguousarray(c[:, V8_KEY, V8_CH]).view(np.uint8)


def unpack_v4(rec):
    return _unpack4(rec, V8_KEY, V8_CH)


def pack_v4(codes):
    return _pack4(codes, V8_KEY, V8_CH)


def unpack_v16(rec):
    """V16 records -> fp16 bit patterns [N, 64, 128]."""
    r = np.ascontiguousarray(rec).view(np.uint16).reshape(-1, 8192)
    out = np.empty((r.shape[0], BN, D), np.uint16)
    out[:, V16_KEY, V16_CH] = r
    return out


def pack_v16(bits):
    c = np.asarray(bits, np.uint16).reshape(-1, BN, D)
    return np.ascontiguousarray(c[:, V16_KEY, V16_CH])
