"""Frames between the HTTP process and its GPU worker over a Unix socketpair.

The message set and header follow the reference's worker protocol
(src/worker_ipc.h:14-68): a 12-byte little-endian header

    [u32 type][u32 payload length][u32 request id]

then the payload: JSON, or JSON with binary parts so that embeddings and
image files do not pass through JSON text,

    floats: [u32 json length][json][f32 values]
    blobs:  [u32 json length][json] then per blob [u32 length][bytes]

A reply carries the request id of its request; ERR replaces any reply.
"""
import enum
import json
import struct

import numpy as np

HEADER = struct.Struct("<III")
MAX_PAYLOAD = 256 << 20  # 256 MiB, as the reference's cap
_U32 = struct.Struct("<I")


class Frame(enum.IntEnum):
    HELLO = 0x01                   # worker -> parent {"pid", "role"}
    LOAD_REQ = 0x10                # parent -> worker load config
    LOAD_RESP = 0x11               # {"ok", "error", "hidden_size", "max_position_embeddings"}
    ENCODE_IMAGES_REQ = 0x20       # blobs {"pooling", "max_num_patches", "return_last_hidden"}
    ENCODE_IMAGES_RESP = 0x21      # floats {"n", "dim"}
    ENCODE_TEXT_REQ = 0x22         # {"prompts"}
    ENCODE_TEXT_RESP = 0x23        # floats {"n", "dim"}
    CLASSIFY_REQ = 0x24            # blobs {"prompts", "max_num_patches", "return_logits"}
    CLASSIFY_RESP = 0x25           # {"scores", "logits"?}
    CLASSIFY_FROM_EMB_REQ = 0x26   # floats {"prompts", "return_logits", "n", "dim"}
    CLASSIFY_FROM_EMB_RESP = 0x27  # {"scores", "logits"?}
    ERR = 0x2F                     # {"error"}
    PING = 0x40
    PONG = 0x41
    SHUTDOWN = 0xFF


class FrameError(Exception):
    """kind: "eof" (closed between frames), "eof-mid-frame", "too-big",
    "protocol", "socket" or "timeout"."""

    def __init__(self, kind, msg=""):
        super().__init__(f"{kind}: {msg}" if msg else kind)
        self.kind = kind


def _recv_exact(sock, n, allow_clean_eof=False):
    buf = bytearray(n)
    view = memoryview(buf)
    got = 0
    while got < n:
        try:
            r = sock.recv_into(view[got:], n - got)
        except TimeoutError as e:
            raise FrameError("timeout", str(e)) from e
        except OSError as e:
            raise FrameError("socket", str(e)) from e
        if r == 0:
            raise FrameError("eof" if (got == 0 and allow_clean_eof) else "eof-mid-frame")
        got += r
    return bytes(buf)


def _as_bytes(payload):
    if payload is None:
        return b""
    if isinstance(payload, (bytes, bytearray, memoryview)):
        return bytes(payload)
    if isinstance(payload, str):
        return payload.encode()
    return json.dumps(payload).encode()


def send_frame(sock, ftype, req_id, payload=None):
    data = _as_bytes(payload)
    if len(data) > MAX_PAYLOAD:
        raise FrameError("too-big", f"{len(data)} bytes")
    try:
        sock.sendall(HEADER.pack(int(ftype), len(data), req_id) + data)
    except TimeoutError as e:
        raise FrameError("timeout", str(e)) from e
    except OSError as e:
        raise FrameError("socket", str(e)) from e


def recv_frame(sock):
    """(type, request id, payload bytes); FrameError("eof") when the peer
    closed between frames."""
    ftype, n, req_id = HEADER.unpack(_recv_exact(sock, HEADER.size, allow_clean_eof=True))
    if n > MAX_PAYLOAD:
        raise FrameError("too-big", f"{n} bytes")
    return ftype, req_id, _recv_exact(sock, n) if n else b""


def as_json(payload):
    try:
        return json.loads(payload.decode() or "{}")
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise FrameError("protocol", f"bad JSON payload: {e}") from e


def _split_meta(payload):
    if len(payload) < 4:
        raise FrameError("protocol", "payload shorter than its JSON length word")
    (n,) = _U32.unpack_from(payload, 0)
    if 4 + n > len(payload):
        raise FrameError("protocol", "JSON length past the payload")
    return as_json(payload[4:4 + n]), 4 + n


def pack_floats(meta, values):
    j = json.dumps(meta).encode()
    return _U32.pack(len(j)) + j + np.ascontiguousarray(values, np.float32).tobytes()


def unpack_floats(payload):
    meta, off = _split_meta(payload)
    if (len(payload) - off) % 4:
        raise FrameError("protocol", "float part not a whole number of f32")
    return meta, np.frombuffer(payload, np.float32, offset=off).copy()


def pack_blobs(meta, blobs):
    j = json.dumps(meta).encode()
    parts = [_U32.pack(len(j)), j]
    for b in blobs:
        parts += [_U32.pack(len(b)), bytes(b)]
    return b"".join(parts)


def unpack_blobs(payload):
    meta, off = _split_meta(payload)
    blobs = []
    while off < len(payload):
        if off + 4 > len(payload):
            raise FrameError("protocol", "truncated blob length")
        (n,) = _U32.unpack_from(payload, off)
        off += 4
        if off + n > len(payload):
            raise FrameError("protocol", "blob past the payload")
        blobs.append(payload[off:off + n])
        off += n
    return meta, blobs
