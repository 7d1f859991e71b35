"""Damaged copies of a GGML model file (test helper): truncations at the
header, the first tensor record and the data, and corrupted header fields and
first-record fields, each as (what, bytes)."""
import struct


def first_record(data: bytes) -> int:
    """Offset of the first tensor record: [n_dims, name_len, type, ne...,
    name], the first place after the fixed header where such a record with a
    printable dotted name parses."""
    for o in range(16, min(len(data) - 64, 4096), 4):
        nd, nl, ty = struct.unpack_from("<iii", data, o)
        if not (1 <= nd <= 4 and 1 <= nl <= 256 and ty in (0, 1, 2, 3, 8)):
            continue
        ne = struct.unpack_from(f"<{nd}i", data, o + 12)
        if min(ne) <= 0:
            continue
        name = data[o + 12 + 4 * nd:o + 12 + 4 * nd + nl]
        if len(name) == nl and b"." in name and all(32 < c < 127 for c in name):
            return o
    raise AssertionError("no tensor record found")


def damaged(data: bytes):
    rec = first_record(data)
    nd = struct.unpack_from("<i", data, rec)[0]
    name_end = rec + 12 + 4 * nd + struct.unpack_from("<i", data, rec + 4)[0]
    cases = []
    for cut in sorted({0, 3, 8, 15, 40, rec - 1, rec + 5, name_end - 1, name_end + 40, len(data) // 2, len(data) - 1}):
        cases.append((f"truncated_at_{cut}", data[:cut]))

    def patch(off, value, what):
        b = bytearray(data)
        struct.pack_into("<i", b, off, value)
        cases.append((what, bytes(b)))

    patch(0, 0x12345678, "magic")
    patch(4, 99, "version")
    patch(8, 42, "ftype")
    patch(12, -1, "n_tensors_negative")
    patch(12, 1 << 30, "n_tensors_huge")
    patch(12, 3, "n_tensors_short")
    for v in (0, 5, -1):
        patch(rec, v, f"n_dims_{v}")
    for v in (0, 300, 1 << 30, -4):
        patch(rec + 4, v, f"name_len_{v}")
    for v in (7, 99, -1):
        patch(rec + 8, v, f"type_{v}")
    for v in (0, -5, 0x7FFFFFFF):
        patch(rec + 12, v, f"ne0_{v}")
    patch(rec + 12 + 4 * (nd - 1), 0x40000000, "ne_last_huge")
    return cases
