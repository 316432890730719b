"""Tree gather cases shared by the oracle and GPU tests: injective layouts of
JustFitTreeGatherParams (TreeVerify.h:54-69), random 16-bit data, paths that
ascend with path[i] >= i (padded with the last row, as jf_accept_tree writes
them) and retained counts 0..8, plus the closed form the in-place copy must
equal: row i := original row path[i] for i < retained, other rows
unchanged."""
import numpy as np


def _gather_layout(rng, lanes, layers, rows, columns, inner, inner_stride, outer_stride, pad):
    row_stride = (columns // inner) * outer_stride if inner < columns else columns * inner_stride
    row_stride = max(row_stride, inner * inner_stride) + pad
    lane_stride = rows * row_stride + pad
    layer_stride = lanes * lane_stride + pad
    units = layers * layer_stride + pad
    return dict(columns=columns, inner=inner, inner_stride=inner_stride, outer_stride=outer_stride,
                row_stride=row_stride, lane_stride=lane_stride, layer_stride=layer_stride,
                layers=layers, lanes=lanes, rows=rows), units


def gather_case(rng, lanes=5, layers=3, rows=16, columns=40, inner=40, inner_stride=1,
                outer_stride=0, pad=3):
    p, units = _gather_layout(rng, lanes, layers, rows, columns, inner, inner_stride,
                              outer_stride or inner * inner_stride, pad)
    data = rng.integers(0, 65536, units, dtype=np.uint64).astype(np.uint16)
    path = np.zeros((lanes, 8), np.uint32)
    retained = rng.integers(0, 9, lanes).astype(np.uint32)
    for b in range(lanes):
        cur = 0
        for i in range(8):  # ascending, path[i] >= i, padded with the last row
            if i:
                cur = min(rows - 1, max(cur + 1, i + int(rng.integers(0, 3))))
            path[b, i] = cur
    return data, path, retained, p


def gather_closed_form(data, path, retained, p):
    out = data.copy()
    for b in range(p["lanes"]):
        for y in range(p["layers"]):
            for c in range(p["columns"]):
                base = (y * p["layer_stride"] + b * p["lane_stride"] + (c // p["inner"]) * p["outer_stride"]
                        + (c % p["inner"]) * p["inner_stride"])
                for i in range(min(int(retained[b]), 8)):
                    out[base + i * p["row_stride"]] = data[base + int(path[b, i]) * p["row_stride"]]
    return out


