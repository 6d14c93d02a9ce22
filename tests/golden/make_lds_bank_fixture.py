"""Patterns for lds_bank_probe.hip and the fixture made from its counters.

    python3 make_lds_bank_fixture.py patterns        -> lds_bank_patterns.txt, lds_bank_labels.json
    python3 make_lds_bank_fixture.py fixture CSV     -> lds_bank_probe_gfx950.json

Pattern groups (one probe dispatch each):
  E1  two active lanes a < b, lane b at byte offset 256 (the same banks as
      lane a's offset 0, another address): a conflict means the two lanes
      are served in the same pass.  Lane 0 against every lane, and every
      lane against each single-bit flip of its index; per op.
  E2  lanes (0, 2^j) with the second lane at offset X: which X share banks
      (reads: every pair; writes: the pairs one pass serves).
  E3  whole-wave patterns of the GEMM kernels' LDS accesses.
"""
import csv
import collections
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OPS = {0: "rd128", 1: "rd64", 2: "rdtr64", 3: "wr128", 4: "wr64"}
ALL = (1 << 64) - 1


def v7_a(lane, s2):
    """Version 7's A fragment read (f16_pingpong.hip, pp16): row lane % 16
    of a 128-byte-row half-tile, chunk 4 s2 + lane / 16, XOR (row / 2) % 8."""
    row, chunk = lane & 15, 4 * s2 + (lane >> 4)
    return row * 128 + 16 * (chunk ^ ((row >> 1) & 7))


def v7_flush(lane, q):
    """Version 7's fp16 epilogue read: 8 rows x 8 chunk pairs per instruction."""
    row, ch = 8 * q + (lane >> 3), lane & 7
    return row * 128 + 16 * (ch ^ ((row >> 1) & 7))


def v8_a(lane, swz):
    """Version 8's A fragment read (f16_skinny_sk.hip): row lane % 16 of a
    64-byte-row block, chunk lane / 16, XOR swz(row)."""
    row, chunk = lane & 15, lane >> 4
    return row * 64 + 16 * (chunk ^ swz(row))


def v8_b(lane, wavecols, cg, c, h):
    """Version 8's B transpose read (128-column blocks, 256-byte k-rows):
    lane 16g + 4jj + q names k-row 8g + jj + 4h, chunk (wavecols / 8) cg +
    2c + q / 2 XOR 2 (k % 4) ^ 8 bit3(k), half q % 2."""
    g, jj, q = lane >> 4, (lane >> 2) & 3, lane & 3
    krow = 8 * g + jj + 4 * h
    chunk = (wavecols // 8) * cg + 2 * c + (q >> 1)
    return krow * 256 + 16 * (chunk ^ ((2 * (krow & 3)) ^ (((krow >> 3) & 1) << 3))) + 8 * (q & 1)


def v7_b(lane, gw, j):
    """Version 7's B transpose read (512-byte k-rows), k-step 0, half 0."""
    g, jj, q = lane >> 4, (lane >> 2) & 3, lane & 3
    krow = 8 * g + jj
    c = gw * 8 + 2 * j + (q >> 1)
    swz = [0, 6, 12, 10][krow & 3] ^ (((krow >> 3) & 1) << 1)
    return krow * 512 + 16 * (c ^ swz) + 8 * (q & 1)


def v11_epi_h(lane, i, j, swz):
    """Version 11's fp16 epilogue staging write (f16_pp128.hip Epi<half>):
    block (i, j), lane l -> row 16 i + l % 16, 8-byte unit 4 j + l / 16 of a
    64-byte row, placed at unit ^ swz(row)."""
    row, unit = 16 * i + (lane & 15), 4 * j + (lane >> 4)
    return row * 64 + 8 * (unit ^ swz(row))


def v11_epi_f(lane, i, j, swz):
    """Version 11's fp32 epilogue staging write (Epi<float>): row 16 i +
    l % 16, 16-byte chunk 4 j + l / 16 of a 128-byte row, at chunk ^ swz(row)."""
    row, chunk = 16 * i + (lane & 15), 4 * j + (lane >> 4)
    return row * 128 + 16 * (chunk ^ swz(row))


def v11_epi_f_read(lane, q, swz):
    """Version 11's fp32 epilogue read: 8 rows x 8 chunks per instruction."""
    row, ch = 8 * q + (lane >> 3), lane & 7
    return row * 128 + 16 * (ch ^ swz(row))


def v7_epi_h(lane, i, j):
    """Version 7's fp16 staging write (f16_pingpong.hip epi16_unit_addr):
    128-byte rows of 16 units, unit u of row r at u ^ (r % 16)."""
    row, unit = 16 * i + (lane & 15), 4 * j + (lane >> 4)
    return row * 128 + 8 * (unit ^ (row & 15))


def v7_epi_f(lane, i, j):
    """Version 7's fp32 staging write (Epi16<float>): 256-byte rows, chunk ^ (r % 16)."""
    row, chunk = 16 * (i & 3) + (lane & 15), 4 * j + (lane >> 4)
    return row * 256 + 16 * (chunk ^ (row & 15))


def v3_epi_h(lane, i, j, g4):
    """Versions 2/3's fp16 staging write (f16_dma.hip): 256-byte rows, 16-byte
    chunk 4 j + g4 ^ (r % 16), 8-byte half l / 32."""
    row, chunk, hsel = 32 * i + (lane & 31), 4 * j + g4, lane >> 5
    return row * 256 + 16 * (chunk ^ (row & 15)) + 8 * hsel


V11_EPI_H = {"swz 2((r>>2)&3)": lambda r: ((r >> 2) & 3) << 1, "swz (r>>1)&7": lambda r: (r >> 1) & 7}
V11_EPI_F = {"swz (r>>1)&7": lambda r: (r >> 1) & 7, "swz r&7": lambda r: r & 7}


V8_SWIZZLES = {
    "swz(row>>2)&3": lambda r: (r >> 2) & 3,
    "unswizzled": lambda r: 0,
    "swz r&3": lambda r: r & 3,
    "swz (r>>1)&3": lambda r: (r >> 1) & 3,
}


def patterns():
    cfgs = []

    def add(label, op, mask, offs):
        assert len(offs) == 64 and all(0 <= o <= 65536 - 16 for o in offs)
        cfgs.append((label, op, mask, offs))

    for op in OPS:
        pairs = set((0, l) for l in range(1, 64))
        for l in range(64):
            for j in range(6):
                m = l ^ (1 << j)
                pairs.add((min(l, m), max(l, m)))
        for a, b in sorted(pairs):
            o = [0] * 64
            o[b] = 256
            add(f"E1 {OPS[op]} pair {a} {b}", op, (1 << a) | (1 << b), o)
    for op, step in ((0, 16), (1, 8), (2, 8)):
        for pr in ((0, 1), (0, 2), (0, 4), (0, 8), (0, 16), (0, 32)):
            for x in range(step, 1024 + step, step):
                o = [0] * 64
                o[pr[1]] = x
                add(f"E2 {OPS[op]} lanes {pr[0]} {pr[1]} X {x}", op, (1 << pr[0]) | (1 << pr[1]), o)
    for op, step, prs in ((3, 16, ((0, 1), (0, 2), (0, 4))), (4, 8, ((0, 1), (0, 2), (0, 4), (0, 8)))):
        for pr in prs:
            for x in range(step, 1024 + step, step):
                o = [0] * 64
                o[pr[1]] = x
                add(f"E2 {OPS[op]} lanes {pr[0]} {pr[1]} X {x}", op, (1 << pr[0]) | (1 << pr[1]), o)
    for s2 in (0, 1):
        add(f"E3 rd128 v7A s2={s2}", 0, ALL, [v7_a(l, s2) for l in range(64)])
    for q in (0, 1):
        add(f"E3 rd128 v7flush q={q}", 0, ALL, [v7_flush(l, q) for l in range(64)])
    for name, f in V8_SWIZZLES.items():
        add(f"E3 rd128 v8A {name}", 0, ALL, [v8_a(l, f) for l in range(64)])
    add("E3 rd128 linear", 0, ALL, [16 * l for l in range(64)])
    for wc, ncg, ncb in ((32, 4, 2), (64, 2, 4)):
        for cg in range(ncg):
            for c in range(ncb):
                for h in (0, 1):
                    add(f"E3 rdtr64 v8B wavecols={wc} cg={cg} c={c} h={h}", 2, ALL,
                        [v8_b(l, wc, cg, c, h) for l in range(64)])
    for gw in range(4):
        for j in range(4):
            add(f"E3 rdtr64 v7B gw={gw} j={j}", 2, ALL, [v7_b(l, gw, j) for l in range(64)])
    for name, f in V11_EPI_H.items():
        for j in (0, 1):
            add(f"E3 wr64 v11epiH {name} j={j}", 4, ALL, [v11_epi_h(l, 0, j, f) for l in range(64)])
    for name, f in V11_EPI_F.items():
        for j in (0, 1):
            add(f"E3 wr128 v11epiF {name} j={j}", 3, ALL, [v11_epi_f(l, 0, j, f) for l in range(64)])
        add(f"E3 rd128 v11epiFread {name} q=0", 0, ALL, [v11_epi_f_read(l, 0, f) for l in range(64)])
    for j in (0, 1):
        add(f"E3 wr64 v7epiH j={j}", 4, ALL, [v7_epi_h(l, 0, j) for l in range(64)])
        add(f"E3 wr128 v7epiF j={j}", 3, ALL, [v7_epi_f(l, 0, j) for l in range(64)])
    add("E3 wr64 v3epiH j=0 g4=0", 4, ALL, [v3_epi_h(l, 0, 0, 0) for l in range(64)])
    add("E3 wr64 linear", 4, ALL, [8 * l for l in range(64)])
    add("E3 wr128 linear", 3, ALL, [16 * l for l in range(64)])
    return cfgs


def write_patterns():
    cfgs = patterns()
    with open(os.path.join(HERE, "lds_bank_patterns.txt"), "w") as f:
        for _, op, mask, offs in cfgs:
            f.write(f"{op} {mask:x} " + " ".join(map(str, offs)) + "\n")
    json.dump([c[0] for c in cfgs], open(os.path.join(HERE, "lds_bank_labels.json"), "w"))
    print(len(cfgs), "patterns")


def write_fixture(csv_path):
    labels = json.load(open(os.path.join(HERE, "lds_bank_labels.json")))
    per = collections.OrderedDict()
    for r in csv.DictReader(open(csv_path)):
        if "probe" not in r["Kernel_Name"]:
            continue
        d = per.setdefault(int(r["Dispatch_Id"]), {})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    vals = list(per.values())
    assert len(vals) == len(labels), (len(vals), len(labels))
    out = {"source": "lds_bank_probe.hip on one MI355X (gfx950); values per instruction "
                     "(SQ_LDS_BANK_CONFLICT / 16, SQ_LDS_IDX_ACTIVE / 16)",
           "pairs_rd128": [], "pairs_rd64": [], "pairs_wr128": [], "pairs_wr64": [], "patterns": [],
           "xsweep_rd128": [], "xsweep_rd64": [], "xsweep_rdtr64": [], "xsweep_wr128": [], "xsweep_wr64": []}
    for lab, v in zip(labels, vals):
        p = lab.split()
        conf, act = v["SQ_LDS_BANK_CONFLICT"] / 16, v["SQ_LDS_IDX_ACTIVE"] / 16
        if p[0] == "E1" and p[1] in ("rd128", "rd64", "wr128", "wr64"):
            out["pairs_" + p[1]].append([int(p[3]), int(p[4]), conf])
        elif p[0] == "E2":
            out["xsweep_" + p[1]].append([int(p[4]), int(p[6]), conf])
        elif p[0] == "E3":
            out["patterns"].append([" ".join(p[1:]), conf, act])
    json.dump(out, open(os.path.join(HERE, "lds_bank_probe_gfx950.json"), "w"), indent=0)


if __name__ == "__main__":
    if sys.argv[1] == "patterns":
        write_patterns()
    else:
        write_fixture(sys.argv[2])
