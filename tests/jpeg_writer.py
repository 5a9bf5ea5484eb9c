"""A small baseline JPEG writer (ITU-T T.81) for the decoder tests, with the
decode it implies.

`encode` writes a baseline sequential JPEG (SOF0, Huffman) of an 8-bit
greyscale or RGB image with chosen sampling factors, quality, restart
interval, interleaved or one-component-per-scan layout, and Huffman tables
built from the data's own symbol counts (optionally made deep, so that some
codes are longer than 9 bits).  It returns the file's bytes and the
quantised coefficients it coded, from which `ideal_decode` computes the
samples a decoder following T.81 A.3.3 (a float64 inverse DCT rounded to the
nearest level), the triangle-filter chroma upsampling and the JFIF colour
conversion must produce.  This module is test infrastructure only.
"""
import heapq
import struct

import numpy as np

ZZ = np.array([0, 1, 8, 16, 9, 2, 3, 10, 17, 24, 32, 25, 18, 11, 4, 5, 12, 19, 26, 33, 40, 48,
               41, 34, 27, 20, 13, 6, 7, 14, 21, 28, 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15,
               23, 30, 37, 44, 51, 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62,
               63])

# T.81 Annex K.1 example quantisation tables (natural order), scaled by quality
QL = np.array([16, 11, 10, 16, 24, 40, 51, 61, 12, 12, 14, 19, 26, 58, 60, 55, 14, 13, 16, 24,
               40, 57, 69, 56, 14, 17, 22, 29, 51, 87, 80, 62, 18, 22, 37, 56, 68, 109, 103, 77,
               24, 35, 55, 64, 81, 104, 113, 92, 49, 64, 78, 87, 103, 121, 120, 101, 72, 92, 95,
               98, 112, 100, 103, 99])
QC = np.array([17, 18, 24, 47, 99, 99, 99, 99, 18, 21, 26, 66, 99, 99, 99, 99, 24, 26, 56, 99,
               99, 99, 99, 99, 47, 66, 99, 99, 99, 99, 99, 99] + [99] * 32)


def qtable(base, quality):
    s = 5000 // quality if quality < 50 else 200 - 2 * quality
    return np.clip((base * s + 50) // 100, 1, 255).astype(np.int64)


def _cos():
    x = np.arange(8)
    c = np.cos((2 * x[:, None] + 1) * x[None, :] * np.pi / 16) * 0.5
    c[:, 0] *= np.sqrt(0.5)
    return c  # c[x][u] = C(u)/2 cos((2x+1) u pi / 16)


CS = _cos()


def fdct(block):
    return CS.T @ (block - 128.0) @ CS  # F[v][u]


def idct(coef):
    return CS @ coef @ CS.T


def rgb_to_ycc(rgb):
    r, g, b = [rgb[..., i].astype(np.float64) for i in range(3)]
    y = 0.299 * r + 0.587 * g + 0.114 * b
    cb = -0.168736 * r - 0.331264 * g + 0.5 * b + 128
    cr = 0.5 * r - 0.418688 * g - 0.081312 * b + 128
    return [np.clip(np.floor(p + 0.5), 0, 255) for p in (y, cb, cr)]


def huff_lengths(freq, deep=False):
    """code lengths (<= 16) from symbol counts by Huffman's procedure, with
    T.81 K.2's reserved symbol (no all-ones code) and length limiting"""
    syms = sorted(freq)
    f = {s: freq[s] for s in syms}
    if deep:  # a skewed distribution: long codes for the rare symbols
        f = {s: (1 << 20) >> min(i, 19) for i, s in enumerate(sorted(syms, key=lambda s: -freq[s]))}
    f[256] = 0  # reserved, least frequent
    heap = [(max(v, 1) if k != 256 else 0, i, [k]) for i, (k, v) in enumerate(f.items())]
    heapq.heapify(heap)
    size = {k: 0 for k in f}
    n = len(heap)
    while len(heap) > 1:
        a, _, sa = heapq.heappop(heap)
        b, _, sb = heapq.heappop(heap)
        for s in sa + sb:
            size[s] += 1
        n += 1
        heapq.heappush(heap, (a + b, n, sa + sb))
    if len(f) == 1:
        size = {k: 1 for k in f}
    bits = [0] * 33
    for s, l in size.items():
        bits[l] += 1
    for i in range(32, 16, -1):  # K.2 adjust_bits
        while bits[i] > 0:
            j = i - 2
            while bits[j] == 0:
                j -= 1
            bits[i] -= 2
            bits[i - 1] += 1
            bits[j + 1] += 2
            bits[j] -= 1
    i = 16
    while bits[i] == 0:
        i -= 1
    bits[i] -= 1  # drop the reserved symbol
    order = sorted((s for s in f if s != 256), key=lambda s: (size[s], s))
    counts = bits[1:17]
    vals = order
    codes, code, k = {}, 0, 0
    for l in range(1, 17):
        for _ in range(counts[l - 1]):
            codes[vals[k]] = (code, l)
            code += 1
            k += 1
        code <<= 1
    return counts, vals, codes


class Bits:
    def __init__(self):
        self.out = bytearray()
        self.acc = 0
        self.n = 0

    def put(self, v, n):
        for i in range(n - 1, -1, -1):
            self.acc = (self.acc << 1) | ((v >> i) & 1)
            self.n += 1
            if self.n == 8:
                self.out.append(self.acc)
                if self.acc == 0xFF:
                    self.out.append(0)
                self.acc = 0
                self.n = 0

    def flush(self):
        while self.n:
            self.put(1, 1)


def category(v):
    return int(abs(v)).bit_length()


def bits_of(v, s):
    return v if v >= 0 else v + (1 << s) - 1


def encode(img, quality=90, sampling=((1, 1), (1, 1), (1, 1)), restart=0, interleaved=True,
           deep=False, adobe_rgb=False, q16=False):
    """img: uint8 [H][W] or [H][W][3].  Returns (bytes, info) where info holds
    per component: sampling, quant table, coefficient blocks [by][bx][8][8]
    (quantised, natural order) and the plane size."""
    img = np.asarray(img)
    H, W = img.shape[:2]
    if img.ndim == 2:
        planes, sampling = [img.astype(np.float64)], sampling[:1]
    elif adobe_rgb:
        planes = [img[..., i].astype(np.float64) for i in range(3)]
    else:
        planes = rgb_to_ycc(img)
    nc = len(planes)
    hmax = max(s[0] for s in sampling)
    vmax = max(s[1] for s in sampling)
    mcux, mcuy = -(-W // (8 * hmax)), -(-H // (8 * vmax))
    qs = [qtable(QL, quality), qtable(QC, quality)]
    comps = []
    for i, p in enumerate(planes):
        h, v = sampling[i]
        # downsample by averaging (fx x fy boxes), padded by edge replication
        fx, fy = hmax // h, vmax // v
        pw, ph = mcux * 8 * hmax, mcuy * 8 * vmax
        full = np.pad(p, ((0, ph - H), (0, pw - W)), mode="edge")
        small = full.reshape(ph // fy, fy, pw // fx, fx).mean(axis=(1, 3))
        small = np.clip(np.floor(small + 0.5), 0, 255)
        xw, yh = -(-W * h // hmax), -(-H * v // vmax)
        # samples past the component's own size repeat its last row / column
        small[:, xw:] = small[:, xw - 1:xw]
        small[yh:, :] = small[yh - 1:yh, :]
        q = qs[0 if i == 0 or adobe_rgb else 1]
        bh, bw = small.shape[0] // 8, small.shape[1] // 8
        blocks = np.zeros((bh, bw, 8, 8), np.int64)
        for by in range(bh):
            for bx in range(bw):
                F = fdct(small[by * 8:by * 8 + 8, bx * 8:bx * 8 + 8])
                blocks[by, bx] = np.floor(F / q.reshape(8, 8) + 0.5)
        comps.append(dict(h=h, v=v, q=q, blocks=blocks, xw=xw, yh=yh, tq=0 if q is qs[0] else 1,
                          id=(ord("RGB"[i]) if adobe_rgb else i + 1)))
    # symbol statistics per table (DC table 0/1, AC table 0/1)
    th = [0 if (i == 0 or adobe_rgb) else 1 for i in range(nc)]
    order = []  # (component, block y, block x) in coding order, with restart marks

    def units(ci_list):
        if len(ci_list) == 1:
            c = comps[ci_list[0]]
            ux, uy = -(-c["xw"] // 8), -(-c["yh"] // 8)
            for y in range(uy):
                for x in range(ux):
                    yield [(ci_list[0], y, x)]
        else:
            for my in range(mcuy):
                for mx in range(mcux):
                    u = []
                    for ci in ci_list:
                        c = comps[ci]
                        for by in range(c["v"]):
                            for bx in range(c["h"]):
                                u.append((ci, my * c["v"] + by, mx * c["h"] + bx))
                    yield u

    scans = [list(range(nc))] if interleaved else [[i] for i in range(nc)]
    dcf, acf = [dict(), dict()], [dict(), dict()]
    for sc in scans:
        for k, u in enumerate(units(sc)):
            if restart and k % restart == 0:
                pred = {ci: 0 for ci in sc}
            elif k == 0:
                pred = {ci: 0 for ci in sc}
            for ci, by, bx in u:
                z = comps[ci]["blocks"][by, bx].reshape(64)[ZZ]
                d = int(z[0]) - pred[ci]
                pred[ci] = int(z[0])
                dcf[th[ci]][category(d)] = dcf[th[ci]].get(category(d), 0) + 1
                run = 0
                last = max([i for i in range(1, 64) if z[i] != 0], default=0)
                for i in range(1, last + 1):
                    if z[i] == 0:
                        run += 1
                        continue
                    while run > 15:
                        acf[th[ci]][0xF0] = acf[th[ci]].get(0xF0, 0) + 1
                        run -= 16
                    s = (run << 4) | category(int(z[i]))
                    acf[th[ci]][s] = acf[th[ci]].get(s, 0) + 1
                    run = 0
                if last < 63:
                    acf[th[ci]][0] = acf[th[ci]].get(0, 0) + 1
    tabs = {}
    for t in range(2):
        if dcf[t]:
            tabs[("dc", t)] = huff_lengths(dcf[t], deep)
        if acf[t]:
            tabs[("ac", t)] = huff_lengths(acf[t], deep)
    out = bytearray(b"\xff\xd8")

    def seg(marker, payload):
        out.extend(struct.pack(">BBH", 0xFF, marker, len(payload) + 2))
        out.extend(payload)

    seg(0xE0, b"JFIF\x00\x01\x01\x00\x00\x01\x00\x01\x00\x00")
    if adobe_rgb:
        seg(0xEE, b"Adobe\x00\x64\x00\x00\x00\x00\x00")
    for t in sorted({c["tq"] for c in comps}):
        q = qs[t]
        if q16:
            seg(0xDB, bytes([0x10 | t]) + b"".join(struct.pack(">H", int(q[ZZ[k]])) for k in range(64)))
        else:
            seg(0xDB, bytes([t]) + bytes(int(q[ZZ[k]]) for k in range(64)))
    sof = struct.pack(">BHHB", 8, H, W, nc)
    for c in comps:
        sof += struct.pack(">BBB", c["id"], (c["h"] << 4) | c["v"], c["tq"])
    seg(0xC0, sof)
    for (kind, t), (counts, vals, _) in sorted(tabs.items()):
        seg(0xC4, bytes([(0 if kind == "dc" else 0x10) | t]) + bytes(counts) + bytes(vals))
    if restart:
        seg(0xDD, struct.pack(">H", restart))
    for sc in scans:
        sos = bytes([len(sc)])
        for ci in sc:
            sos += bytes([comps[ci]["id"], (th[ci] << 4) | th[ci]])
        seg(0xDA, sos + b"\x00\x3f\x00")
        bw = Bits()
        rst = 0
        for k, u in enumerate(units(sc)):
            if restart and k % restart == 0:
                if k:
                    bw.flush()
                    bw.out.extend(bytes([0xFF, 0xD0 + (rst & 7)]))
                    rst += 1
                pred = {ci: 0 for ci in sc}
            elif k == 0:
                pred = {ci: 0 for ci in sc}
            for ci, by, bx in u:
                dcc = tabs[("dc", th[ci])][2]
                acc = tabs[("ac", th[ci])][2]
                z = comps[ci]["blocks"][by, bx].reshape(64)[ZZ]
                d = int(z[0]) - pred[ci]
                pred[ci] = int(z[0])
                s = category(d)
                bw.put(*dcc[s])
                bw.put(bits_of(d, s), s)
                run = 0
                last = max([i for i in range(1, 64) if z[i] != 0], default=0)
                for i in range(1, last + 1):
                    if z[i] == 0:
                        run += 1
                        continue
                    while run > 15:
                        bw.put(*acc[0xF0])
                        run -= 16
                    s = category(int(z[i]))
                    bw.put(*acc[(run << 4) | s])
                    bw.put(bits_of(int(z[i]), s), s)
                    run = 0
                if last < 63:
                    bw.put(*acc[0])
        bw.flush()
        out.extend(bw.out)
    out.extend(b"\xff\xd9")
    return bytes(out), dict(comps=comps, W=W, H=H, hmax=hmax, vmax=vmax, adobe_rgb=adobe_rgb)


def _clamp_round(x):
    return np.clip(np.floor(x + 0.5), 0, 255)


def _up2(a, axis):
    """2x along an axis: (3*nearest + next), edges replicated (x4 scale)"""
    n = a.shape[axis]
    idx = np.arange(n)
    lo = np.take(a, np.maximum(idx - 1, 0), axis=axis)
    hi = np.take(a, np.minimum(idx + 1, n - 1), axis=axis)
    even, odd = 3 * a + lo, 3 * a + hi
    out = np.stack([even, odd], axis=axis + 1)
    shape = list(a.shape)
    shape[axis] = 2 * n
    return out.reshape(shape)


def ideal_decode(info):
    """the samples a T.81 decoder with a float64 IDCT (rounded to nearest),
    triangle-filter 2x upsampling and JFIF colour conversion outputs:
    uint8 [H][W] or [H][W][3]"""
    W, H, hmax, vmax = info["W"], info["H"], info["hmax"], info["vmax"]
    full = []
    for c in info["comps"]:
        bh, bw = c["blocks"].shape[:2]
        pl = np.zeros((bh * 8, bw * 8))
        q = c["q"].reshape(8, 8)
        for by in range(bh):
            for bx in range(bw):
                pl[by * 8:by * 8 + 8, bx * 8:bx * 8 + 8] = _clamp_round(
                    idct(c["blocks"][by, bx] * q) + 128)
        pl = pl[:c["yh"], :c["xw"]].astype(np.int64)
        fx, fy = hmax // c["h"], vmax // c["v"]
        sh = 0
        if fx == 2:
            pl = _up2(pl, 1)
            sh += 2
        if fy == 2:
            pl = _up2(pl, 0)
            sh += 2
        if sh:
            pl = (pl + (1 << (sh - 1))) >> sh
        pl = np.pad(pl, ((0, max(0, H - pl.shape[0])), (0, max(0, W - pl.shape[1]))), mode="edge")
        full.append(pl[:H, :W].astype(np.float64))
    if len(full) == 1:
        return full[0].astype(np.uint8)
    if info["adobe_rgb"]:
        return np.stack(full, axis=-1).astype(np.uint8)
    y, cb, cr = full[0], full[1] - 128, full[2] - 128
    r = _clamp_round(y + 1.402 * cr)
    g = _clamp_round(y - 0.344136 * cb - 0.714136 * cr)
    b = _clamp_round(y + 1.772 * cb)
    return np.stack([r, g, b], axis=-1).astype(np.uint8)
