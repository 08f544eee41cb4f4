"""Deployment loading for the ``fa`` op group: offline build with a metadata
sidecar, validated precompiled load, fail-closed dispatcher ownership.

Mirrors the reference's ``CustomOps.build`` / ``load_precompiled`` / ``load``
contract (__init__.py:654-1011) for this build's artifact, a C-ABI HIP library
opened with ctypes (the torch op is registered from Python over it):

* ``FAOps().build(out_dir)`` compiles ``libmi355_fa.so`` for gfx950 into
  ``out_dir`` and publishes ``libmi355_fa.so.json`` next to it (schema contract,
  offload targets, runtime compatibility, source/toolchain fingerprints,
  library SHA-256 and size). It never loads what it builds and refuses to
  overwrite a library already loaded in this process.
* ``FAOps().load_precompiled(path)`` validates the sidecar against this Python
  wrapper and the running process BEFORE opening the library (missing,
  tampered or incompatible artifacts raise ``CustomOpsError``; nothing falls
  back to compiling), then opens it, checks the ABI and exported symbols,
  registers ``recsys_ops::mha_fwd_with_mask`` and verifies its schema and Meta
  kernel before reporting the group available.
* ``load()`` is the development path: the in-tree library, compiled by hipcc
  when missing and ``allow_jit`` is True. With ``allow_jit=False`` it only
  accepts a group already loaded by ``load_precompiled``.

One library per process owns the operator: loading a different file (another
build, or a copy of the same bytes) for the same operator, or an operator that
another library already registered, raises instead of replacing it.
"""
from __future__ import annotations

import fcntl
import hashlib
import json
import os
import re
import subprocess
import tempfile
import threading
from pathlib import Path
from typing import Optional

import torch

from . import _lib, build as _build, fa

METADATA_VERSION = 1
PRODUCER = "custom_ops_amd"

_LOCK = threading.RLock()
_LIBRARIES: dict = {}    # identity -> record
_OP_OWNERS: dict = {}    # "ns::op" -> identity


class CustomOpsError(RuntimeError):
    """Load/build failure (the reference's exception type name, __init__.py:71)."""


def _json_hash(value) -> str:
    return hashlib.sha256(json.dumps(value, sort_keys=True).encode()).hexdigest()


def _metadata_fingerprint(metadata: dict) -> str:
    return _json_hash({k: v for k, v in metadata.items()
                       if k not in ("build_fingerprint", "library")})


def _file_sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def _file_stat(path: Path) -> tuple:
    st = path.stat()
    return (st.st_dev, st.st_ino, st.st_size, st.st_mtime_ns)


def _library_identity(path: Path) -> tuple:
    """(device, inode, sha256): the same file with the same bytes."""
    st = _file_stat(path)
    return (st[0], st[1], _file_sha256(path)), st


def _runtime_compatibility() -> dict:
    """What a library built here needs from the process that loads it."""
    hip = getattr(torch.version, "hip", None) or ""
    return {
        "abi_version": _lib.ABI_VERSION,
        "torch": ".".join(torch.__version__.split("+")[0].split(".")[:2]),
        "hip_major": hip.split(".")[0] if hip else "",
    }


def _canonical_archs(value) -> list:
    """Sorted unique gfx targets; rejects anything that is not 'gfx' + digits/letters."""
    items = value.split(";") if isinstance(value, str) else list(value)
    out = sorted({s.strip() for s in items if str(s).strip()})
    for a in out:
        if not re.fullmatch(r"gfx[0-9a-f]{3,4}", a):
            raise CustomOpsError(f"invalid offload target {a!r} (expected e.g. 'gfx950')")
    return out


def _visible_archs() -> set:
    """gfx names of the visible GPUs (empty without a GPU)."""
    if not torch.cuda.is_available():
        return set()
    return {torch.cuda.get_device_properties(i).gcnArchName.split(":")[0]
            for i in range(torch.cuda.device_count())}


def _has_schema(qualified: str) -> bool:
    try:
        return bool(torch._C._jit_get_schemas_for_operator(qualified))
    except RuntimeError:
        return False


def _schema(qualified: str) -> str:
    schemas = torch._C._jit_get_schemas_for_operator(qualified)
    return str(schemas[0]) if schemas else ""


def _hipcc_version(hipcc: str) -> str:
    try:
        out = subprocess.run([hipcc, "--version"], capture_output=True, text=True, timeout=60)
        for line in out.stdout.splitlines():
            if "version" in line.lower():
                return line.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return ""


class FAOps:
    """The ``fa`` op group (reference ``FAOps``, recsys.py:165-202)."""

    namespace = fa.NAMESPACE
    so_name = "libmi355_fa"
    required_ops = [fa.OP_NAME]
    fake_ops = [fa.OP_NAME]
    op_schemas = {fa.OP_NAME: fa.SCHEMA}
    build_version = "1"
    default_offload_arch = "gfx950"

    def __init__(self, *, allow_jit: bool = True) -> None:
        self._loaded = False
        self._load_error: Optional[str] = None
        self._library_path: Optional[Path] = None
        self._metadata_path: Optional[Path] = None
        self._allow_jit = True
        self.configure(allow_jit=allow_jit)

    # ── policy ──────────────────────────────────────────────────────────────
    @property
    def allow_jit(self) -> bool:
        """Whether load() may compile the in-tree library (hipcc)."""
        return self._allow_jit

    @allow_jit.setter
    def allow_jit(self, value: bool) -> None:
        self.configure(allow_jit=value)

    def configure(self, *, allow_jit: bool) -> "FAOps":
        if not isinstance(allow_jit, bool):
            raise TypeError("allow_jit must be a bool")
        with _LOCK:
            self._allow_jit = allow_jit
        return self

    def disable_jit(self) -> "FAOps":
        return self.configure(allow_jit=False)

    @property
    def library_path(self) -> Optional[Path]:
        return self._library_path if self._loaded else None

    @property
    def metadata_path(self) -> Optional[Path]:
        return self._metadata_path if self._loaded else None

    def is_available(self) -> bool:
        return self._loaded

    def load_error(self) -> Optional[str]:
        return self._load_error

    # ── offline build ───────────────────────────────────────────────────────
    def _schema_contract(self) -> dict:
        return {f"{self.namespace}::{k}": f"{self.namespace}::{v}"
                for k, v in sorted(self.op_schemas.items())}

    def _build_inputs(self, offload_arch, extra_flags) -> dict:
        archs = _canonical_archs(offload_arch or self.default_offload_arch)
        if not archs:
            raise CustomOpsError("no offload target given")
        flags = [f for f in _build.HIPCC_FLAGS if not f.startswith("--offload-arch=")]
        extra = list(extra_flags)
        for f in extra:
            if not isinstance(f, str) or not f.strip() or "\n" in f:
                raise CustomOpsError(f"invalid extra flag {f!r}")
        return {"offload_arch": archs, "flags": flags, "extra_flags": extra,
                "sources": [os.path.relpath(_build.SRC, _build.REPO_DIR)],
                "include_dirs": [os.path.relpath(_build.INCLUDE, _build.REPO_DIR)]}

    @staticmethod
    def _source_fingerprint(inputs: dict) -> str:
        h = hashlib.sha256(json.dumps(inputs, sort_keys=True).encode())
        for rel in inputs["sources"]:
            h.update(Path(_build.REPO_DIR, rel).read_bytes())
        for rel in inputs["include_dirs"]:
            for hdr in sorted(Path(_build.REPO_DIR, rel).glob("*.h")):
                h.update(hdr.name.encode())
                h.update(hdr.read_bytes())
        return h.hexdigest()

    def build(self, output_directory, *, offload_arch: Optional[str] = None,
              extra_flags=(), verbose: bool = False) -> Path:
        """Compile and export ``<so_name>.so`` + ``<so_name>.so.json`` without loading.

        hipcc cross-compiles, so this runs on a host without a GPU. Both files
        must be deployed together."""
        with _LOCK:
            inputs = self._build_inputs(offload_arch, extra_flags)
            fingerprint = self._source_fingerprint(inputs)
            hipcc = _build.hipcc()
            out = Path(output_directory).expanduser().resolve()
            out.mkdir(parents=True, exist_ok=True)
            library = out / f"{self.so_name}.so"
            sidecar = library.with_suffix(library.suffix + ".json")
            metadata = {
                "format_version": METADATA_VERSION,
                "producer": PRODUCER,
                "namespace": self.namespace,
                "so_name": self.so_name,
                "build_version": self.build_version,
                "compatibility": _runtime_compatibility(),
                "offload_arch": inputs["offload_arch"],
                "required_ops": sorted(self.required_ops),
                "fake_ops": sorted(self.fake_ops),
                "schemas": self._schema_contract(),
                "schema_fingerprint": _json_hash(self._schema_contract()),
                "source_fingerprint": fingerprint,
                "build": {**inputs, "toolchain": {"hipcc": _hipcc_version(hipcc)}},
            }
            metadata["build_fingerprint"] = _metadata_fingerprint(metadata)
            with (out / f"{self.so_name}.lock").open("a") as lock:
                fcntl.flock(lock, fcntl.LOCK_EX)
                try:
                    if library.exists() and any(
                            rec["identity"][:2] == _file_stat(library)[:2]
                            for rec in _LIBRARIES.values()):
                        raise CustomOpsError(
                            f"cannot overwrite a library loaded in this process: {library}")
                    with tempfile.TemporaryDirectory(prefix=f".{self.so_name}-build-",
                                                     dir=out) as work:
                        product = Path(work) / library.name
                        cmd = [hipcc, *inputs["flags"],
                               *[f"--offload-arch={a}" for a in inputs["offload_arch"]],
                               *inputs["extra_flags"],
                               *[f"-I{Path(_build.REPO_DIR, d)}" for d in inputs["include_dirs"]],
                               *[str(Path(_build.REPO_DIR, s)) for s in inputs["sources"]],
                               "-o", str(product)]
                        if verbose:
                            print(" ".join(cmd), flush=True)
                        res = subprocess.run(cmd, capture_output=True, text=True)
                        if res.returncode != 0:
                            raise CustomOpsError(f"hipcc failed ({res.returncode}):\n"
                                                 f"{res.stderr[-4000:]}")
                        if self._source_fingerprint(inputs) != fingerprint:
                            raise CustomOpsError("sources changed during the build; nothing exported")
                        metadata["library"] = {"filename": library.name,
                                               "sha256": _file_sha256(product),
                                               "size": product.stat().st_size}
                        pending = Path(work) / "metadata.json"
                        pending.write_text(json.dumps(metadata, sort_keys=True, indent=2) + "\n")
                        os.replace(product, library)
                        os.replace(pending, sidecar)
                finally:
                    fcntl.flock(lock, fcntl.LOCK_UN)
            return library

    # ── precompiled load ────────────────────────────────────────────────────
    def _validate_metadata(self, library: Path, sidecar: Path) -> tuple:
        try:
            metadata = json.loads(sidecar.read_text())
        except (OSError, ValueError) as e:
            raise CustomOpsError(f"unreadable metadata {sidecar}: {e}") from e
        if not isinstance(metadata, dict):
            raise CustomOpsError("precompiled metadata must be a JSON object")
        expected = {"format_version": METADATA_VERSION, "producer": PRODUCER,
                    "namespace": self.namespace, "so_name": self.so_name,
                    "build_version": self.build_version}
        for key, value in expected.items():
            if metadata.get(key) != value or type(metadata.get(key)) is not type(value):
                raise CustomOpsError(f"precompiled {key} mismatch: built={metadata.get(key)!r}, "
                                     f"expected={value!r}")
        compat = metadata.get("compatibility")
        if not isinstance(compat, dict):
            raise CustomOpsError("precompiled compatibility information is missing")
        for key, value in _runtime_compatibility().items():
            if compat.get(key) != value or type(compat.get(key)) is not type(value):
                raise CustomOpsError(f"precompiled compatibility mismatch ({key}): "
                                     f"built={compat.get(key)!r}, runtime={value!r}")
        for key, ops in (("required_ops", self.required_ops), ("fake_ops", self.fake_ops)):
            vals = metadata.get(key)
            if not isinstance(vals, list) or sorted(vals) != sorted(ops):
                raise CustomOpsError(f"precompiled {key} mismatch: built={vals}, "
                                     f"expected={sorted(ops)}")
        if metadata.get("schemas") != self._schema_contract():
            raise CustomOpsError("precompiled schema contract does not match this Python wrapper")
        if metadata.get("schema_fingerprint") != _json_hash(self._schema_contract()):
            raise CustomOpsError("precompiled schema fingerprint is invalid")
        for key in ("source_fingerprint", "build_fingerprint"):
            if not isinstance(metadata.get(key), str) or not re.fullmatch(r"[0-9a-f]{64}",
                                                                         metadata[key]):
                raise CustomOpsError(f"precompiled {key} is missing or invalid")
        if metadata["build_fingerprint"] != _metadata_fingerprint(metadata):
            raise CustomOpsError("precompiled build fingerprint is invalid")
        targets = metadata.get("offload_arch")
        if not isinstance(targets, list) or not targets or targets != _canonical_archs(targets):
            raise CustomOpsError("precompiled offload targets are missing or noncanonical")
        visible = _visible_archs()
        if not visible.issubset(targets):
            raise CustomOpsError(f"precompiled target mismatch: visible={sorted(visible)}, "
                                 f"built={targets}")
        binary = metadata.get("library")
        if not isinstance(binary, dict) or binary.get("filename") != library.name:
            raise CustomOpsError("precompiled library identity information is missing")
        if type(binary.get("size")) is not int or binary["size"] <= 0:
            raise CustomOpsError("precompiled library size is invalid")
        identity, stat = _library_identity(library)
        if binary.get("sha256") != identity[2] or binary["size"] != stat[2]:
            raise CustomOpsError(f"precompiled library hash/size mismatch: {library}")
        return metadata, identity, stat

    def _operator_names(self) -> set:
        return {f"{self.namespace}::{n}" for n in set(self.required_ops) | set(self.op_schemas)}

    def _check_conflicts(self, identity: tuple, names: set) -> None:
        for rec in _LIBRARIES.values():
            if rec["identity"][:2] == identity[:2] and rec["identity"] != identity:
                raise CustomOpsError("an already loaded library file was modified; "
                                     "use a fresh process")
        rec = _LIBRARIES.get(identity)
        if rec is not None and rec["error"] is not None:
            raise CustomOpsError("this library previously failed after loading started; use a "
                                 "fresh process. " + rec["error"])
        for name in names:
            owner = _OP_OWNERS.get(name)
            if owner is not None and owner != identity:
                raise CustomOpsError(f"dispatcher library conflict for {name}: already owned by "
                                     f"{_LIBRARIES[owner]['path']}; use a fresh process")
            if owner is None and _has_schema(name):
                raise CustomOpsError(f"dispatcher operator {name} is already registered by an "
                                     "untracked library; use a fresh process")

    def _open(self, library: Path, identity: tuple) -> dict:
        names = self._operator_names()
        self._check_conflicts(identity, names)
        rec = _LIBRARIES.get(identity)
        if rec is not None and rec["ready"]:
            return rec
        rec = {"identity": identity, "path": library, "names": names, "ready": False,
               "error": None}
        _LIBRARIES[identity] = rec          # reserve before opening
        for name in names:
            _OP_OWNERS[name] = identity
        try:
            _lib.load(str(library))
            fa.register()
        except Exception as e:
            rec["error"] = str(e)
            raise
        return rec

    def _finish(self, rec: dict) -> None:
        for name, schema in self._schema_contract().items():
            got = _schema(name)
            if got != schema:
                rec["error"] = f"registered schema {got!r} != contract {schema!r}"
                raise CustomOpsError(rec["error"])
        for op in self.fake_ops:
            if not torch._C._dispatch_has_kernel_for_dispatch_key(f"{self.namespace}::{op}",
                                                                   "Meta"):
                rec["error"] = f"fake/Meta implementation missing for {self.namespace}::{op}"
                raise CustomOpsError(rec["error"])
        rec["ready"] = True
        self._library_path = rec["path"]
        self._load_error = None
        self._loaded = True

    def load_precompiled(self, library_path, metadata_path=None) -> "FAOps":
        """Validate, then load a deployment library; disables implicit compiling.

        The default sidecar is ``<library_path>.json``."""
        with _LOCK:
            self._allow_jit = False
            self._loaded = False
            try:
                library = Path(library_path).expanduser().resolve(strict=True)
                if not library.is_file():
                    raise CustomOpsError(f"precompiled library is not a file: {library}")
                sidecar = (Path(metadata_path).expanduser() if metadata_path is not None
                           else Path(str(Path(library_path).expanduser()) + ".json"))
                sidecar = sidecar.resolve(strict=True)
                _, identity, stat = self._validate_metadata(library, sidecar)
                if _file_stat(library) != stat:
                    raise CustomOpsError(f"library changed during validation: {library}")
                rec = self._open(library, identity)
                self._finish(rec)
                self._metadata_path = sidecar
            except Exception as e:
                self._loaded = False
                self._load_error = str(e)
                raise CustomOpsError(f"[FAOps] precompiled load failed (JIT disabled): {e}") from e
        return self

    # ── development load ────────────────────────────────────────────────────
    def load(self) -> "FAOps":
        """In-tree library; compiled with hipcc when missing and allow_jit is True."""
        with _LOCK:
            if self._loaded:
                return self
            if not self._allow_jit:
                self._load_error = ("JIT is disabled for FAOps; call load_precompiled("
                                    "library_path, metadata_path=None) before load()")
                raise CustomOpsError(self._load_error)
            try:
                path = Path(_build.lib_path())
                if not path.exists():
                    _build.build()
                path = path.resolve(strict=True)
                identity, _ = _library_identity(path)
                rec = self._open(path, identity)
                self._finish(rec)
                self._metadata_path = None
            except Exception as e:
                self._loaded = False
                self._load_error = str(e)
                raise CustomOpsError(f"[FAOps] load failed: {e}") from e
        return self
