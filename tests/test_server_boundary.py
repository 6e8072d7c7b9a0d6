"""The protocol boundary on the CPU: handshake and request validation of the
MI355X server need no device.  Where the reference CPU server has been built
(oracle/_ref, from the reference sources), the same malformed requests must be
rejected with the same messages."""
import struct

import pytest

import oracle
from cpde_amd import wire
from cpde_amd.build import SERVER

BAD_REQUESTS = [
    (42, b''),                                        # unknown command
    (2, b'\x01\x00'),                                 # truncated fields
    (2, struct.pack('<iiii', 1, 1, 1, 0)),            # variable count 0
    (2, struct.pack('<iiii', 0, 1, 1, 1)),            # empty dimensions
    (4, struct.pack('<QQi', 5, 6, 0)),                # unknown handles
    (11, struct.pack('<iQ', 7, 1)),                   # invalid object kind
    (1, b'x'),                                        # trailing fields
    (3, wire.encode(('i32[]', [2, 1]), ('i32[]', [0, 1]))),  # input layer not linear
    (3, wire.encode(('i32[]', [2]), ('i32[]', [1]))),        # too few layers
]


def server_path():
    if not SERVER.exists():
        pytest.skip('protocol server not built')
    return SERVER


def errors(executable):
    out = []
    with wire.Session(executable) as s:
        for op, body in BAD_REQUESTS:
            try:
                s.request(op, body)
                out.append(None)
            except wire.ServerError as e:
                out.append(str(e))
    return out


def test_handshake():
    with wire.Session(server_path()) as s:
        assert (s.protocol, s.version) == ('CPDE/3', 6)
        # diagnostics | graphs | expressions | RPROP restore | wrapper initialisation,
        # without the CPU-backend and host-probe bits (the client reports 'cuda')
        assert s.capabilities == 31


def test_rejections_keep_the_server_usable():
    msgs = errors(server_path())
    assert all(m is not None for m in msgs), msgs
    assert msgs[0] == 'unknown command' and msgs[1] == 'truncated command'


def test_rejections_match_the_reference_server():
    ref = oracle.reference_server()
    if ref is None:
        pytest.skip('reference CPU server not built (make -C oracle ref)')
    assert errors(server_path()) == errors(ref)


def test_frame_with_invalid_size_ends_the_session():
    with wire.Session(server_path()) as s:
        s.send_raw(struct.pack('<Q', 2))  # length below the 4-byte kind
        with pytest.raises(RuntimeError):
            s.receive(timeout=30)
