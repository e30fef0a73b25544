"""Index construction primitives on the GPU: the gofann_build_* C ABI over
torch device tensors (torch holds device memory only; every computation is
a HIP kernel of libgofann_hip.so).

`index.py` composes these into the label graphs, the coarse k-means and
the PQ / RaBitQ encoders; the reference composes cuVS CAGRA, PQ and
IVF-RaBitQ for the same artifacts (src/index/graph_builder.cu:1279-1315,
tools/quantization/pq_builder.cu:49-153,
third_party/cuvs_rabitq/src/neighbors/ivf_rabitq/gpu_index/
quantizer_gpu_fast.cu:39-265).

A backend object has this interface (the CPU oracle's restatement,
oracle/pyoracle.py OracleBuild, has the same one, so the build orchestration
can be checked step for step):
  rows(x)                              matrix the backend computes on
  take(rows, idx)                      rows idx (host int array) in order
  host(a) / dev(a)                     to a numpy array / to the backend
  assign(rows, centres)                nearest centre per row (u32)
  kmeanspp(rows, k, seed), kmeans(rows, centres, iters)
  knn(rows, bucket_off, k, probe_off, probe)
  bucket_reps(rows, bucket_off)        (means, reps)
  medoid(rows)                         int
  links(knn, bucket_of, reps, near, order, **params)   graph [n][R] (host)
  cagra_optimize(knn, degree)          (pruned, graph) in the sorted space
  reach(graph, entry)                  (reached bool host array, count)
  pq_train(rows, centroids, pq_dim, iters), pq_encode(rows, centroids, pq_dim)
  rotate(rows, rotation)               rows x rotation (f32)
  rabitq_encode(rotated, anchors)      (anchor ids, codes, factors)
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib

_ELEM = {torch.uint8: _lib.ELEM_U8, torch.float32: _lib.ELEM_F32, torch.float16: _lib.ELEM_F16}


def _u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


class HipBuild:
    """gofann_build_* on one device, through a gofann context."""

    def __init__(self, ctx: _lib.Context | None = None, device: str = "cuda"):
        self.ctx = ctx if ctx is not None else _lib.Context(0)
        self.lib = self.ctx.lib
        self.device = torch.device(device)

    # -- arrays ----------------------------------------------------------
    def rows(self, x) -> torch.Tensor:
        if isinstance(x, np.ndarray):
            x = torch.from_numpy(x)
        if x.dtype not in _ELEM:
            x = x.float()
        return x.to(self.device).contiguous()

    def take(self, rows: torch.Tensor, idx) -> torch.Tensor:
        ix = torch.as_tensor(np.ascontiguousarray(idx, dtype=np.int64), device=rows.device)
        return rows.index_select(0, ix).contiguous()

    def host(self, a) -> np.ndarray:
        if isinstance(a, torch.Tensor):
            a = a.cpu().numpy()
        return np.asarray(a)

    def dev(self, a, dtype=None) -> torch.Tensor:
        if isinstance(a, np.ndarray):
            if a.dtype == np.uint32:
                a = a.view(np.int32)
            a = torch.from_numpy(np.ascontiguousarray(a))
        t = a.to(self.device)
        if dtype is not None:
            t = t.to(dtype)
        return t.contiguous()

    def _elem(self, rows: torch.Tensor) -> int:
        return _ELEM[rows.dtype]

    def _check(self, rc):
        self.ctx.check(rc)

    # -- primitives ------------------------------------------------------
    def assign(self, rows: torch.Tensor, centres) -> torch.Tensor:
        c = self.dev(centres, torch.float32)
        out = torch.empty(rows.shape[0], dtype=torch.int32, device=self.device)
        self._check(self.lib.gofann_build_assign(self.ctx.handle, rows.data_ptr(), self._elem(rows),
                                                 rows.shape[1], rows.shape[0], c.data_ptr(),
                                                 c.shape[0], out.data_ptr(), None))
        return out

    def kmeanspp(self, rows: torch.Tensor, k: int, seed: int) -> torch.Tensor:
        out = torch.empty(k, rows.shape[1], dtype=torch.float32, device=self.device)
        self._check(self.lib.gofann_build_kmeanspp(self.ctx.handle, rows.data_ptr(),
                                                   self._elem(rows), rows.shape[1], rows.shape[0],
                                                   k, seed, out.data_ptr()))
        return out

    def kmeans(self, rows: torch.Tensor, centres, iters: int) -> torch.Tensor:
        c = self.dev(centres, torch.float32).clone()
        self._check(self.lib.gofann_build_kmeans(self.ctx.handle, rows.data_ptr(), self._elem(rows),
                                                 rows.shape[1], rows.shape[0], c.shape[0], iters,
                                                 c.data_ptr()))
        return c

    def knn(self, rows: torch.Tensor, bucket_off, k: int, probe_off=None, probe=None) -> torch.Tensor:
        bo = self.dev(np.asarray(bucket_off, np.uint32))
        po = self.dev(np.asarray(probe_off, np.uint32)) if probe_off is not None else None
        pb = self.dev(np.asarray(probe, np.uint32)) if probe is not None else None
        n = int(np.asarray(bucket_off)[-1])
        out = torch.empty(n, k, dtype=torch.int32, device=self.device)
        b = _lib.BuildBuckets(bo.data_ptr(), len(bucket_off) - 1, n, _lib.ptr(po), _lib.ptr(pb))
        self._check(self.lib.gofann_build_knn(self.ctx.handle, rows.data_ptr(), self._elem(rows),
                                              rows.shape[1], C.byref(b), k, out.data_ptr(), None))
        return out

    def bucket_reps(self, rows: torch.Tensor, bucket_off):
        bo = self.dev(np.asarray(bucket_off, np.uint32))
        nb = len(bucket_off) - 1
        means = torch.empty(nb, rows.shape[1], dtype=torch.float32, device=self.device)
        reps = torch.empty(nb, dtype=torch.int32, device=self.device)
        self._check(self.lib.gofann_build_bucket_reps(self.ctx.handle, rows.data_ptr(),
                                                      self._elem(rows), rows.shape[1],
                                                      bo.data_ptr(), nb, means.data_ptr(),
                                                      reps.data_ptr()))
        return means, reps

    def medoid(self, rows: torch.Tensor) -> int:
        out = C.c_uint32()
        self._check(self.lib.gofann_build_medoid(self.ctx.handle, rows.data_ptr(), self._elem(rows),
                                                 rows.shape[1], rows.shape[0], C.byref(out)))
        return int(out.value)

    def links(self, knn, bucket_of, reps, near, order, degree, local, near_links, rep_local,
              rep_near, entry, seed) -> np.ndarray:
        n = len(bucket_of)
        knn_t = self.dev(knn) if knn is not None else None
        bo = self.dev(np.asarray(bucket_of, np.uint32))
        rp = self.dev(reps)
        nr = self.dev(near)
        od = self.dev(np.asarray(order, np.uint32))
        out = torch.empty(n, degree, dtype=torch.int32, device=self.device)
        inp = _lib.BuildLinkInputs(n, _lib.ptr(knn_t), knn_t.shape[1] if knn_t is not None else 0,
                                   bo.data_ptr(), rp.data_ptr(), nr.data_ptr(),
                                   nr.shape[1] if nr.dim() == 2 else 0, rp.shape[0], od.data_ptr())
        prm = _lib.BuildLinkParams(degree, local, near_links, rep_local, rep_near,
                                   0xFFFFFFFF if entry is None else int(entry), int(seed))
        self._check(self.lib.gofann_build_links(self.ctx.handle, C.byref(inp), C.byref(prm),
                                                out.data_ptr()))
        return _u32(out)

    def cagra_optimize(self, knn, degree: int):
        k = self.dev(knn)
        n, kin = k.shape
        pruned = torch.empty(n, degree, dtype=torch.int32, device=self.device)
        out = torch.empty(n, degree, dtype=torch.int32, device=self.device)
        self._check(self.lib.gofann_build_cagra_optimize(self.ctx.handle, k.data_ptr(), n, kin,
                                                         degree, pruned.data_ptr(),
                                                         out.data_ptr()))
        return pruned, out

    def reach(self, graph, entry: int):
        g = self.dev(graph)
        n, deg = g.shape
        reached = torch.empty(n, dtype=torch.int32, device=self.device)
        cnt = C.c_uint32()
        self._check(self.lib.gofann_build_reach(self.ctx.handle, g.data_ptr(), n, deg, int(entry),
                                                reached.data_ptr(), C.byref(cnt)))
        return reached.cpu().numpy() != 0, int(cnt.value)

    def pq_train(self, rows: torch.Tensor, centroids, pq_dim: int, iters: int) -> torch.Tensor:
        c = self.dev(centroids, torch.float32).clone()
        self._check(self.lib.gofann_build_pq_train(self.ctx.handle, rows.data_ptr(),
                                                   self._elem(rows), rows.shape[1], rows.shape[0],
                                                   pq_dim, iters, c.data_ptr()))
        return c

    def pq_encode(self, rows: torch.Tensor, centroids, pq_dim: int) -> torch.Tensor:
        c = self.dev(centroids, torch.float32)
        out = torch.empty(rows.shape[0], pq_dim, dtype=torch.uint8, device=self.device)
        self._check(self.lib.gofann_build_pq_encode(self.ctx.handle, rows.data_ptr(),
                                                    self._elem(rows), rows.shape[1],
                                                    rows.shape[0], pq_dim, c.data_ptr(),
                                                    out.data_ptr(), pq_dim))
        return out

    def rotate(self, rows: torch.Tensor, rotation) -> torch.Tensor:
        r = self.dev(rotation, torch.float32)
        out = torch.empty(rows.shape[0], r.shape[1], dtype=torch.float32, device=self.device)
        self._check(self.lib.gofann_build_rotate(self.ctx.handle, rows.data_ptr(), self._elem(rows),
                                                 rows.shape[1], rows.shape[0], r.data_ptr(),
                                                 r.shape[1], out.data_ptr()))
        return out

    def rabitq_encode(self, rotated: torch.Tensor, anchors):
        a = self.dev(anchors, torch.float32)
        n, P = rotated.shape
        aid = torch.empty(n, dtype=torch.int32, device=self.device)
        codes = torch.empty(n, P // 8, dtype=torch.uint8, device=self.device)
        fac = torch.empty(n, 3, dtype=torch.float32, device=self.device)
        self._check(self.lib.gofann_build_rabitq_encode(self.ctx.handle, rotated.data_ptr(), n, P,
                                                        a.data_ptr(), a.shape[0], aid.data_ptr(),
                                                        codes.data_ptr(), fac.data_ptr()))
        return aid, codes, fac


_default = None


def default_backend() -> HipBuild:
    """The process's GPU build backend (one context on device 0)."""
    global _default
    if _default is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the index build runs on the GPU (gofann_build_*); no GPU is "
                               "visible -- tests on the CPU pass the oracle backend explicitly")
        _default = HipBuild()
    return _default
