"""The mask wire format (Protocol.hpp/Protocol.cpp mask frames, Runtime's
provideMask checks, grammar.rs row rules): host code, run on the CPU. The
expected bytes are written here from the documented layout (a 16-byte
header "SPLH", u16 version 9, u16 type, u64 payload length; little-endian
fields in the order of Protocol.hpp:185-203) and from the offsets the Rust
engine reads (engine.rs:255, 268); the row rules against a direct
restatement of grammar.rs:226-266."""
import struct

import numpy as np
import pytest

import jf_sampler as J


def frame(kind, payload):
    return struct.pack("<4sHHQ", b"SPLH", 9, kind, len(payload)) + payload


def test_mask_request_bytes():
    toks = [5, 248043, 17, 0]
    got = J.mask_request_encode(7, 9, 7760, toks)
    want = frame(0x0103, struct.pack("<QQII", 7, 9, 7760, 4) + struct.pack("<4I", *toks))
    assert got == want
    p = got[16:]  # the engine's reads (engine.rs:255)
    assert struct.unpack_from("<Q", p, 0)[0] == 7 and struct.unpack_from("<I", p, 16)[0] == 7760
    assert len(p) == 24 + 4 * 4
    # The initial-anchor request: no simulation tokens.
    assert J.mask_request_encode(1, 2, 3, []) == frame(0x0103, struct.pack("<QQII", 1, 2, 3, 0))


def test_mask_tree_request_bytes():
    toks, parents = [11, 12, 13, 14, 15], [0, 0, 1, 1, 0]
    got = J.mask_request_encode(3, 4, 7760, toks, parents)
    want = frame(0x0109, struct.pack("<QQII", 3, 4, 7760, 5) + struct.pack("<5I", *toks)
                 + struct.pack("<5I", *parents))
    assert got == want and len(got) - 16 == 24 + 5 * 8  # engine.rs:268


@pytest.mark.parametrize("args", [
    (0, 1, 8, [1]), (1, 0, 8, [1]), (1, 1, 0, [1]), (1, 1, 8, list(range(33))),
    (1, 1, 1 << 20, [1]),
])
def test_mask_request_rejects(args):
    with pytest.raises(J.JfError):
        J.mask_request_encode(*args)


@pytest.mark.parametrize("parents", [[1, 0], [0, 1], [0, 0, 3], []])
def test_mask_tree_request_rejects_parents(parents):
    toks = list(range(max(1, len(parents))))
    with pytest.raises(J.JfError):
        J.mask_request_encode(1, 1, 8, toks[:len(parents)] or [1], parents if parents else [5])


def response(rid, mid, words):
    return frame(0x0003, struct.pack("<QQI", rid, mid, len(words)) + struct.pack(f"<{len(words)}I", *words))


def test_mask_response_decode():
    words = list(np.random.default_rng(0).integers(0, 2**32, 7760 * 3, dtype=np.uint64))
    rid, mid, got = J.mask_response_decode(response(5, 6, words))
    assert (rid, mid) == (5, 6) and np.array_equal(got, np.array(words, np.uint32))


@pytest.mark.parametrize("bad", ["magic", "version", "type", "length", "ids", "empty", "truncated", "count"])
def test_mask_response_rejects(bad):
    f = bytearray(response(5, 6, [1, 2, 3]))
    if bad == "magic":
        f[0] = ord("X")
    elif bad == "version":
        f[4] = 8
    elif bad == "type":
        f[6] = 0x03
        f[7] = 0x01
    elif bad == "length":
        f += b"\0\0\0\0"
    elif bad == "ids":
        f = bytearray(response(0, 6, [1]))
    elif bad == "empty":
        f = bytearray(response(5, 6, []))
    elif bad == "truncated":
        f = bytearray(frame(0x0003, struct.pack("<QQ", 5, 6)))
    elif bad == "count":
        struct.pack_into("<I", f, 16 + 16, 4)
    with pytest.raises(J.JfError):
        J.mask_response_decode(bytes(f))


def test_mask_rows_check():
    W = 4
    rows = np.zeros((3, W), np.uint32)
    rows[:, 1] = 1  # token 32 admitted in every row
    J.mask_rows_check(rows, 3, W)
    J.mask_rows_check(rows, 3, W, pending_token=32)
    with pytest.raises(J.JfError):
        J.mask_rows_check(rows, 3, W, pending_token=33)  # row 0 refuses the anchor
    rows[2] = 0
    with pytest.raises(J.JfError):
        J.mask_rows_check(rows, 3, W)


def test_mask_chain_fill():
    rng = np.random.default_rng(1)
    W, count = 5, 6
    for valid in range(count + 1):
        w = rng.integers(1, 2**32, (count + 1, W), dtype=np.uint64).astype(np.uint32)
        got = J.mask_chain_fill(w, count, valid, W).reshape(count + 1, W)
        want = w.copy()
        want[valid + 1:] = w[valid]
        assert np.array_equal(got, want)


def tree_fill_reference(words, parents, refused):
    """grammar.rs:236-250 restated: states None past a refusal; a None row
    takes rows[parent + 1] (rows[0] for the anchor)."""
    rows = [words[0].copy()]
    alive = []
    for r in range(len(parents)):
        parent_alive = True if r == 0 else alive[parents[r]]
        ok = parent_alive and not refused[r]
        rows.append(words[r + 1].copy() if ok else rows[0 if r == 0 else parents[r] + 1].copy())
        alive.append(ok)
    return np.array(rows)


def test_mask_tree_fill():
    rng = np.random.default_rng(2)
    W = 3
    for _ in range(200):
        n = int(rng.integers(1, 17))
        parents = [0] + [int(rng.integers(0, r)) for r in range(1, n)]
        refused = (rng.random(n) < 0.3).astype(np.uint8)
        w = rng.integers(1, 2**32, (n + 1, W), dtype=np.uint64).astype(np.uint32)
        got = J.mask_tree_fill(w, parents, refused, W).reshape(n + 1, W)
        assert np.array_equal(got, tree_fill_reference(w, parents, refused))
