"""Expert packs: one contiguous, 4 KiB-aligned record per routed expert of one layer.

The format is the reference's derived pack (include/vastloom/inference/deepseek_v4_expert_pack.hpp:
17-77, written by tools/pack_deepseek_experts.py:211-260): a manifest ``vastloom-expert-pack.json``
and a payload ``experts-L<layer>.bin`` beside it. Each manifest record names an expert, its byte
offset and length in the payload (a multiple of the alignment apart), the record's SHA-256, and its
tensors in catalog-bundle order with their offsets inside the record, byte counts, GGML storage
types and shapes. DeepSeek bundles hold ``blk.<layer>.ffn_down_exps.weight.expert.<e>``, then the
gate and up tensors (src/inference/deepseek_v4_graph.cpp:3796-3801); shapes are GGML order
(columns first).

``ExpertPack`` checks the structure (format, alignment, record bounds and overlap, tensor bounds,
the record hashes) and maps the payload read-only; each expert's GGUF bytes are views into that
mapping, ready to be staged into the accelerator's pinned slots. ``write_pack`` writes a pack of
the same format from in-memory experts (the synthetic workloads' experts, for tests and the
residency benchmark). Verifying a pack against a model catalog, as the reference's
verify_deepseek_v4_expert_pack does, needs the checkpoint's catalog and is not part of this path.
"""

from __future__ import annotations

import hashlib
import json
import mmap
from dataclasses import dataclass
from pathlib import Path

import numpy as np

FORMAT = "vastloom.deepseek-v4-expert-pack.v1"
MANIFEST_NAME = "vastloom-expert-pack.json"
PAYLOAD_NAME = "experts-L{layer}.bin"
ALIGNMENT = 4096
MAX_RECORDS = 256
MAX_PAYLOAD_BYTES = 2 * 1024 * 1024 * 1024

PROJECTIONS = ("down", "gate", "up")  # catalog bundle order


class PackError(ValueError):
    pass


@dataclass
class PackTensor:
    name: str
    packed_offset: int
    nbytes: int
    ggml_type: int
    shape: tuple[int, ...]  # GGML order: columns, rows

    @property
    def rows(self) -> int:
        return int(self.shape[1])

    @property
    def cols(self) -> int:
        return int(self.shape[0])


@dataclass
class PackExpert:
    """One record: the expert's gate, up and down matrices as GGUF bytes (views of the payload)."""
    expert: int
    tensors: dict[str, PackTensor]
    data: dict[str, np.ndarray]

    def matrix(self, projection: str) -> tuple[int, int, int, np.ndarray]:
        """(ggml_type, rows, cols, bytes) of 'gate', 'up' or 'down'."""
        t = self.tensors[projection]
        return t.ggml_type, t.rows, t.cols, self.data[projection]


def tensor_name(layer: int, projection: str, expert: int) -> str:
    return f"blk.{layer}.ffn_{projection}_exps.weight.expert.{expert}"


def _projection(name: str) -> str:
    for p in PROJECTIONS:
        if f".ffn_{p}_exps." in name:
            return p
    raise PackError(f"tensor {name!r} is not a routed-expert projection")


def write_pack(root: Path, layer: int, experts: dict[int, dict[str, tuple[int, int, int, np.ndarray]]],
               model_id: str = "synthetic", revision: str = "synthetic") -> dict:
    """Writes a pack of `experts` {id: {'gate'|'up'|'down': (ggml_type, rows, cols, bytes)}}."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    if len(experts) > MAX_RECORDS:
        raise PackError("too many expert records")
    payload_path = root / PAYLOAD_NAME.format(layer=layer)
    records = []
    with payload_path.open("wb") as f:
        for e in sorted(experts):
            offset = f.tell()
            digest = hashlib.sha256()
            tensors = []
            inside = 0
            for p in PROJECTIONS:
                qtype, rows, cols, data = experts[e][p]
                b = np.ascontiguousarray(data, np.uint8).tobytes()
                f.write(b)
                digest.update(b)
                tensors.append({"name": tensor_name(layer, p, e), "packed_offset": inside, "bytes": len(b),
                                "ggml_type": int(qtype), "shape": [int(cols), int(rows)]})
                inside += len(b)
            records.append({"expert": int(e), "offset": offset, "bytes": inside, "sha256": digest.hexdigest(),
                            "source_range_sha256": [], "tensors": tensors})
            f.write(b"\0" * ((-f.tell()) % ALIGNMENT))
        payload_bytes = f.tell()
    if payload_bytes > MAX_PAYLOAD_BYTES:
        raise PackError("pack payload exceeds its safety bound")
    h = hashlib.sha256()
    with payload_path.open("rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    manifest = {"format": FORMAT, "model_id": model_id, "revision": revision, "layer": layer,
                "routing_authority_verified": True, "alignment": ALIGNMENT,
                "payload": {"path": payload_path.name, "bytes": payload_bytes, "sha256": h.hexdigest()},
                "source_artifacts": [], "experts": records}
    (root / MANIFEST_NAME).write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n")
    return manifest


class ExpertPack:
    """A pack mapped read-only: experts by id, their matrices as views of the payload. A pack that
    fails its checks raises PackError and leaves nothing open."""

    experts: dict[int, PackExpert]

    def __init__(self, root: Path, verify_hashes: bool = True):
        root = Path(root)
        m = json.loads((root / MANIFEST_NAME).read_text())
        if m.get("format") != FORMAT:
            raise PackError(f"unsupported pack format {m.get('format')!r}")
        align = int(m.get("alignment", 0))
        if align != ALIGNMENT:
            raise PackError(f"pack alignment {align} is not {ALIGNMENT}")
        self.layer = int(m["layer"])
        payload = m["payload"]
        path = root / payload["path"]
        if path.name != PAYLOAD_NAME.format(layer=self.layer):
            raise PackError(f"payload {path.name!r} does not name layer {self.layer}")
        size = path.stat().st_size
        if size != int(payload["bytes"]) or size > MAX_PAYLOAD_BYTES:
            raise PackError("payload size does not match the manifest")
        self._file = path.open("rb")
        self._map = None
        try:
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ) if size else None
            self._load(m, size, verify_hashes)
        except BaseException:
            self.experts = {}
            self.close()
            raise

    def _load(self, m: dict, size: int, verify_hashes: bool) -> None:
        buf = np.frombuffer(self._map, np.uint8) if size else np.zeros(0, np.uint8)
        records = m.get("experts", [])
        if len(records) > MAX_RECORDS:
            raise PackError("too many expert records")
        self.experts = {}
        end = 0
        for r in sorted(records, key=lambda r: int(r["offset"])):
            e, off, n = int(r["expert"]), int(r["offset"]), int(r["bytes"])
            if off % ALIGNMENT or off < end or off + n > size:
                raise PackError(f"expert {e}: record is misaligned, overlaps or runs past the payload")
            end = off + n
            rec = buf[off:off + n]
            if verify_hashes and hashlib.sha256(rec.tobytes()).hexdigest() != r["sha256"]:
                raise PackError(f"expert {e}: record hash mismatch")
            tensors, data, inside = {}, {}, 0
            for t in r["tensors"]:
                pt = PackTensor(t["name"], int(t["packed_offset"]), int(t["bytes"]), int(t["ggml_type"]),
                                tuple(int(v) for v in t["shape"]))
                if pt.packed_offset != inside or pt.packed_offset + pt.nbytes > n:
                    raise PackError(f"expert {e}: tensor {pt.name} is out of order or out of bounds")
                inside += pt.nbytes
                p = _projection(pt.name)
                tensors[p] = pt
                data[p] = rec[pt.packed_offset:pt.packed_offset + pt.nbytes]
            if set(tensors) != set(PROJECTIONS) or inside != n:
                raise PackError(f"expert {e}: record does not hold exactly gate, up and down")
            if e in self.experts:
                raise PackError(f"expert {e} appears twice")
            self.experts[e] = PackExpert(e, tensors, data)

    def close(self) -> None:
        """Drops the pack's records; the mapping closes once no matrix view handed out remains."""
        self.experts = {}
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:
                pass  # views still reference it; it is released with them
            self._map = None
        self._file.close()
