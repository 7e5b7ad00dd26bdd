"""A PATN wire client (the Mac side of the link, in Python): the message layout of phone-attn.h:74-94 (hdr,
config_req, append_req, attn_req, attn_rep; message numbers of the `msg` enum) and the calls of the reference client
(phone-attn.h:755-785), restated in Python, so a test or a probe can send CONFIG / APPEND / TRUNCATE / ATTN / ATTN_BIG / STATS in any order to a server
such as pa-hip-serve. Pure Python (sockets and numpy); nothing here touches the GPU."""
from __future__ import annotations

import socket
import struct

import numpy as np

MAGIC = 0x4E544150                                   # "PATN"
HELLO, HELLO_OK, CONFIG, APPEND, TRUNCATE, ATTN, ATTN_OK, STATS, OK, ERR, BYE, PING, ATTN_BIG, FETCH = range(1, 15)
NR, HD = 48, 256                                     # query rows per KV head, head dim (phone-attn.h:78-79)


class WireError(RuntimeError):
    pass


class Client:
    def __init__(self, port: int, host: str = "127.0.0.1"):
        self.s = socket.create_connection((host, port), timeout=120)
        self.s.setsockopt(socket.IPPROTO_TCP, socket.TCP_NODELAY, 1)

    def close(self):
        try:
            self._send(BYE, b"")
        finally:
            self.s.close()

    def _send(self, typ: int, *parts: bytes):
        body = b"".join(parts)
        self.s.sendall(struct.pack("<IIQ", MAGIC, typ, len(body)) + body)

    def _recv_exact(self, n: int) -> bytes:
        buf = bytearray()
        while len(buf) < n:
            b = self.s.recv(min(n - len(buf), 1 << 20))
            if not b:
                raise WireError("link closed")
            buf += b
        return bytes(buf)

    def _reply(self, want: int) -> bytes:
        magic, typ, n = struct.unpack("<IIQ", self._recv_exact(16))
        if magic != MAGIC:
            raise WireError("bad magic")
        body = self._recv_exact(n)
        if typ == ERR:
            raise WireError(body.decode(errors="replace"))
        if typ != want:
            raise WireError(f"unexpected reply {typ}")
        return body

    def hello(self) -> str:
        self._send(HELLO)
        body = self._reply(HELLO_OK)
        return body[8:].split(b"\0")[0].decode()

    def config(self, n_layer, nkv, rs, hb, is_q8, gpu_permille=1000, gpu_chunk=1024, store_f16=0, sme_workers=1, sme_helpers=1):
        self._send(CONFIG, struct.pack("<11I", n_layer, nkv, rs, hb, is_q8, sme_workers, sme_helpers, gpu_permille, gpu_chunk,
                                       store_f16, 0))
        self._reply(OK)

    def append(self, layer: int, pos0: int, K: np.ndarray, V: np.ndarray) -> int:
        """K, V: uint8 [n][rs] rows. Returns the keys the layer holds afterwards."""
        n = K.shape[0]
        self._send(APPEND, struct.pack("<III", layer, pos0, n), np.ascontiguousarray(K).tobytes(), np.ascontiguousarray(V).tobytes())
        return struct.unpack("<I", self._reply(OK)[:4])[0]

    def truncate(self, n: int):
        self._send(TRUNCATE, struct.pack("<I", n))
        self._reply(OK)

    def attn(self, layer: int, n_tok: int, nk: int, scale: float, Q: np.ndarray, big: bool = False):
        """Q: uint16 (f16 bits) [ng][nkv][NR][HD]. Returns (rep dict, O f16 bits like Q, lse fp32 [ng][nkv*NR])."""
        Q = np.ascontiguousarray(Q, np.uint16)
        self._send(ATTN_BIG if big else ATTN, struct.pack("<IIIf", layer, n_tok, nk, scale), Q.tobytes())
        body = self._reply(ATTN_OK)
        nk_r, phone_ms, gpu_ms, sme_ms, gpu_pages, pages = struct.unpack("<IfffII", body[:24])
        qn = Q.size
        O = np.frombuffer(body[24:24 + 2 * qn], np.uint16).reshape(Q.shape)
        lse = np.frombuffer(body[24 + 2 * qn:24 + 2 * qn + 4 * (qn // HD)], np.float32)
        return ({"nk": nk_r, "phone_ms": phone_ms, "gpu_ms": gpu_ms, "sme_ms": sme_ms, "gpu_pages": gpu_pages, "pages": pages},
                O, lse)

    def stats(self) -> str:
        self._send(STATS)
        return self._reply(OK).decode(errors="replace")
