"""Host-side rules of the decode-batch projections (no kernel launched): the
split-K part count and argument validation, which return before any HIP
call."""
import ctypes


def test_parts_count(pkg):
    L = pkg._lib.lib()
    # 64 rows: 32 column tiles of 32 -> split K in 8 (256 workgroups).
    assert L.qmi_linear_rows_parts_count(64, 1024, 2048) == 8
    assert L.qmi_linear_rows_parts_count(64, 1024, 3072) == 8
    # 128 rows: 128 tiles of 16 columns -> 2 parts; 256 rows: tiles of 32
    # weight rows for K <= 2048 (128 tiles, 2 parts), of 64 above (64 tiles,
    # 4 parts).
    assert L.qmi_linear_rows_parts_count(128, 1024, 2048) == 2
    assert L.qmi_linear_rows_parts_count(256, 1024, 2048) == 2
    assert L.qmi_linear_rows_parts_count(256, 1024, 3072) == 4
    # Never more parts than 128-element K chunks.
    assert L.qmi_linear_rows_parts_count(1, 16, 128) == 1
    assert L.qmi_linear_rows_parts_count(1, 16, 256) == 2
    # Unsupported shapes: 0.
    for m, n, k in ((0, 1024, 2048), (257, 1024, 2048), (64, 1000, 2048), (64, 1024, 2000)):
        assert L.qmi_linear_rows_parts_count(m, n, k) == 0


def test_validation_before_launch(pkg):
    L = pkg._lib.lib()
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 256)
    null = ctypes.c_void_p(0)
    # NULL inputs, bad shapes and misalignment are rejected without touching memory.
    assert L.qmi_linear_rows(None, 128, None, 128, 4, 16, 128, 0, None, 16, null) != 0
    assert L.qmi_linear_rows(p, 128, p, 128, 300, 16, 128, 0, p, 16, null) != 0
    assert L.qmi_linear_rows(p + 2, 128, p, 128, 4, 16, 128, 0, p, 16, null) != 0
    assert L.qmi_linear_rows(p, 100, p, 128, 4, 16, 128, 0, p, 16, null) != 0
    assert L.qmi_linear_rows_parts(p, 128, p, 128, 4, 16, 256, p, 3, null) != 0  # wrong part count
    assert L.qmi_add_rms_norm_parts(p, 1, 4, p, 16, p, 16, p, p, 16, 12, 1e-6, null) != 0  # n % 8
    assert L.qmi_add_rms_norm_parts(p, 0, 4, p, 16, p, 16, p, p, 16, 16, 1e-6, null) != 0  # no parts
    # m == 0 is a no-op success.
    assert L.qmi_linear_rows(p, 128, p, 128, 0, 16, 128, 0, p, 16, null) == 0
