"""numpy statement of the GEMM operand tile images (the layouts include/afd.h documents):
MXFP4 B images, MXFP8 A images and FP8 images, used by the tests to compare the GPU's packed
bytes with the oracle's codes and scales."""

import numpy as np

IMG_DATA = 16384
IMG_A = IMG_DATA + 128 * 4
IMG_B = IMG_DATA + 256 * 4
SCALE_ORDER = [0, 2, 1, 3]  # physical byte p of a row's scale word holds block SCALE_ORDER[p]


def b_images(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """packed e2m1 [E, N, K/2] + UE8M0 [E, N, K/32] -> images [E, N/256, K/128, IMG_B]."""
    e, n, kb = packed.shape
    k = kb * 2
    nt, kt = n // 256, k // 128
    data = packed.reshape(e, nt, 256, kt, 4, 16).transpose(0, 1, 3, 2, 4, 5)  # e nt kt row chunk byte
    # scale bytes of a row in the order of blocks 0, 2, 1, 3 (a self-inverse permutation)
    sc = scales.reshape(e, nt, 256, kt, 4).transpose(0, 1, 3, 2, 4)[..., SCALE_ORDER]  # e nt kt row
    img = np.zeros((e, nt, kt, IMG_B), dtype=np.uint8)
    body = np.zeros((e, nt, kt, 256, 4, 16), dtype=np.uint8)
    rows = np.arange(256)
    for c in range(4):
        phys = c ^ (((rows >> 1) ^ (rows >> 2)) & 3)
        body[:, :, :, rows, phys, :] = data[:, :, :, rows, c, :]
    img[..., :IMG_DATA] = body.reshape(e, nt, kt, IMG_DATA)
    img[..., IMG_DATA:] = sc.reshape(e, nt, kt, 256 * 4)
    return img


def _swizzle_rows(data: np.ndarray) -> np.ndarray:
    """[..., 256, 4, 16] logical chunks -> the same rows with chunk c at physical chunk
    c ^ ((row >> 1 ^ row >> 2) & 3) (the B image's data layout)."""
    body = np.zeros_like(data)
    rows = np.arange(data.shape[-3])
    for c in range(4):
        phys = c ^ (((rows >> 1) ^ (rows >> 2)) & 3)
        body[..., rows, phys, :] = data[..., rows, c, :]
    return body


def fp8_images(codes: np.ndarray) -> np.ndarray:
    """e4m3 codes [E, N, K] (physical row order) -> FP8 images [E, N/256, K/64, 16384]."""
    e, n, k = codes.shape
    data = codes.reshape(e, n // 256, 256, k // 64, 4, 16).transpose(0, 1, 3, 2, 4, 5)
    return _swizzle_rows(data).reshape(e, n // 256, k // 64, 256 * 64)


def a_rows(images: np.ndarray, k: int):
    """A images [tiles * K/128 * IMG_A] bytes -> (codes [tiles*128, K], scales [tiles*128, K/32])."""
    kt = k // 128
    img = images.reshape(-1, kt, IMG_A)
    tiles = img.shape[0]
    body = img[..., :IMG_DATA].reshape(tiles, kt, 128, 8, 16)
    rows = np.arange(128)
    data = np.zeros((tiles, kt, 128, 8, 16), dtype=np.uint8)
    for c in range(8):
        phys = c ^ ((rows ^ (rows >> 3)) & 7)
        data[:, :, rows, c, :] = body[:, :, rows, phys, :]
    codes = data.transpose(0, 2, 1, 3, 4).reshape(tiles * 128, k)
    sc = img[..., IMG_DATA:].reshape(tiles, kt, 128, 4)[..., SCALE_ORDER]
    sc = sc.transpose(0, 2, 1, 3).reshape(tiles * 128, k // 32)
    return codes, sc
