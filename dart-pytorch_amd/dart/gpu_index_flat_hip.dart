/// MI355X drop-in for `GpuIndexFlat` (lib/core/vector_store/gpu_index_flat.dart)
/// over libvs_hip.so (C ABI: include/vs_hip.h) through `dart:ffi`.
///
/// The vectors stay resident in HBM from `add` on; one native call per
/// `search` returns the k best ids and distances per query, for any k.
/// `rangeSearch` and `removeIds` (which the CUDA-backed class does not
/// support) work, and three helpers cover the other callers of the flat scan:
/// `kmeansStep` (one Lloyd iteration of Kmeans.train, kmeans.dart:91-140),
/// `selfJoin` (the dedup pair list of bin/vector_dedup_demo.dart:115-129) and
/// `GpuIndexFlat.load` (readIndex / readFaissIndex of a flat index file
/// straight into HBM, index_io.dart:8-26, faiss_io.dart:1690-1716).
///
/// This file needs the Dart SDK (absent from the build container); the same
/// call sequence is exercised by the repository's Python tests through the
/// identical C ABI.
library;

import 'dart:ffi' as ffi;
import 'dart:io';
import 'dart:math' as math;
import 'dart:typed_data';

import 'package:ffi/ffi.dart';

import 'index.dart';
import 'index_flat.dart';
import 'kmeans.dart' show KmeansResult;

// ---- C signatures (include/vs_hip.h) --------------------------------------

typedef _CCreate = ffi.Int32 Function(
    ffi.Int32, ffi.Int64, ffi.Int32, ffi.Int32, ffi.Pointer<ffi.Pointer<ffi.Void>>);
typedef _DCreate = int Function(int, int, int, int, ffi.Pointer<ffi.Pointer<ffi.Void>>);
typedef _CDestroy = ffi.Void Function(ffi.Pointer<ffi.Void>);
typedef _DDestroy = void Function(ffi.Pointer<ffi.Void>);
typedef _CAdd = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, ffi.Int32, ffi.Int64);
typedef _DAdd = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, int, int);
typedef _CSearch = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, ffi.Int32,
    ffi.Int64, ffi.Int64, ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Int32>);
typedef _DSearch = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, int, int, int,
    ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Int32>);

final class _RangeC extends ffi.Struct {
  @ffi.Int64()
  external int nq;
  external ffi.Pointer<ffi.Int64> lims;
  external ffi.Pointer<ffi.Float> d;
  external ffi.Pointer<ffi.Int32> i;
}

typedef _CRange = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, ffi.Int32,
    ffi.Int64, ffi.Double, ffi.Pointer<ffi.Pointer<_RangeC>>);
typedef _DRange = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, int, int, double,
    ffi.Pointer<ffi.Pointer<_RangeC>>);
typedef _CRangeFree = ffi.Void Function(ffi.Pointer<_RangeC>);
typedef _DRangeFree = void Function(ffi.Pointer<_RangeC>);
typedef _CRemove = ffi.Int32 Function(
    ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Int64>, ffi.Int64, ffi.Pointer<ffi.Int64>);
typedef _DRemove = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Int64>, int, ffi.Pointer<ffi.Int64>);
typedef _CNtotal = ffi.Int64 Function(ffi.Pointer<ffi.Void>);
typedef _DNtotal = int Function(ffi.Pointer<ffi.Void>);
typedef _CRecon = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Int64, ffi.Int64, ffi.Pointer<ffi.Float>);
typedef _DRecon = int Function(ffi.Pointer<ffi.Void>, int, int, ffi.Pointer<ffi.Float>);
typedef _CErr = ffi.Pointer<Utf8> Function();
typedef _DErr = ffi.Pointer<Utf8> Function();

final class _PairsC extends ffi.Struct {
  @ffi.Int64()
  external int npairs;
  external ffi.Pointer<ffi.Int32> i;
  external ffi.Pointer<ffi.Int32> j;
  external ffi.Pointer<ffi.Float> s;
}

typedef _CJoin = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Double, ffi.Pointer<ffi.Pointer<_PairsC>>);
typedef _DJoin = int Function(ffi.Pointer<ffi.Void>, double, ffi.Pointer<ffi.Pointer<_PairsC>>);
typedef _CPairsFree = ffi.Void Function(ffi.Pointer<_PairsC>);
typedef _DPairsFree = void Function(ffi.Pointer<_PairsC>);
typedef _CKmeans = ffi.Int32 Function(
    ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Float>, ffi.Int64, ffi.Int64, ffi.Pointer<ffi.Double>,
    ffi.Int64, ffi.Pointer<ffi.Int32>, ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Int32>,
    ffi.Pointer<ffi.Double>);
typedef _DKmeans = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Float>, int, int,
    ffi.Pointer<ffi.Double>, int, ffi.Pointer<ffi.Int32>, ffi.Pointer<ffi.Float>,
    ffi.Pointer<ffi.Int32>, ffi.Pointer<ffi.Double>);
typedef _CLoad = ffi.Int32 Function(ffi.Int32, ffi.Pointer<Utf8>, ffi.Int32,
    ffi.Pointer<ffi.Pointer<ffi.Void>>, ffi.Pointer<ffi.Int32>);
typedef _DLoad = int Function(int, ffi.Pointer<Utf8>, int, ffi.Pointer<ffi.Pointer<ffi.Void>>,
    ffi.Pointer<ffi.Int32>);
typedef _CGetI32 = ffi.Int32 Function(ffi.Pointer<ffi.Void>);
typedef _DGetI32 = int Function(ffi.Pointer<ffi.Void>);
typedef _CSubsets = ffi.Int32 Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, ffi.Int32,
    ffi.Int64, ffi.Int64, ffi.Pointer<ffi.Int32>, ffi.Int64, ffi.Pointer<ffi.Int64>,
    ffi.Pointer<ffi.Int64>, ffi.Int64, ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Int32>);
typedef _DSubsets = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Void>, int, int, int,
    ffi.Pointer<ffi.Int32>, int, ffi.Pointer<ffi.Int64>, ffi.Pointer<ffi.Int64>, int,
    ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Int32>);
typedef _CScoreAll = ffi.Int32 Function(
    ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Float>);
typedef _DScoreAll = int Function(ffi.Pointer<ffi.Void>, ffi.Pointer<ffi.Float>, ffi.Pointer<ffi.Float>);

const int _vsOk = 0, _vsInvalid = 1, _vsUnsupported = 4;
const int _dtypeF32 = 0;
const int _storageF32 = 0, _storageAuto = 2;

/// Resolution like cuda_engine.dart:428-455: env override, then
/// <cwd>/native/lib, then next to the executable, then the loader path.
String _findVsLib() {
  final env = Platform.environment['DART_PYTORCH_VS_LIB'];
  if (env != null && env.isNotEmpty) return env;
  const name = 'libvs_hip.so';
  final candidates = <String>['${Directory.current.path}/native/lib/$name'];
  try {
    final exeDir = File(Platform.resolvedExecutable).parent.path;
    candidates
      ..add('$exeDir/native/lib/$name')
      ..add('$exeDir/$name');
  } catch (_) {}
  for (final c in candidates) {
    if (File(c).existsSync()) return c;
  }
  return name;
}

class _Vs {
  _Vs() {
    final lib = ffi.DynamicLibrary.open(_findVsLib());
    create = lib.lookupFunction<_CCreate, _DCreate>('vs_index_create');
    destroy = lib.lookupFunction<_CDestroy, _DDestroy>('vs_index_destroy');
    add = lib.lookupFunction<_CAdd, _DAdd>('vs_index_add');
    search = lib.lookupFunction<_CSearch, _DSearch>('vs_index_search');
    range = lib.lookupFunction<_CRange, _DRange>('vs_index_range_search');
    rangeFree = lib.lookupFunction<_CRangeFree, _DRangeFree>('vs_range_result_free');
    remove = lib.lookupFunction<_CRemove, _DRemove>('vs_index_remove_ids');
    ntotal = lib.lookupFunction<_CNtotal, _DNtotal>('vs_index_ntotal');
    reconstruct = lib.lookupFunction<_CRecon, _DRecon>('vs_index_reconstruct');
    lastError = lib.lookupFunction<_CErr, _DErr>('vs_last_error');
    selfJoin = lib.lookupFunction<_CJoin, _DJoin>('vs_index_self_join');
    pairsFree = lib.lookupFunction<_CPairsFree, _DPairsFree>('vs_pairs_free');
    kmeansStep = lib.lookupFunction<_CKmeans, _DKmeans>('vs_kmeans_step');
    loadFlat = lib.lookupFunction<_CLoad, _DLoad>('vs_index_load_flat');
    indexD = lib.lookupFunction<_CNtotal, _DNtotal>('vs_index_d');
    indexMetric = lib.lookupFunction<_CGetI32, _DGetI32>('vs_index_metric');
    searchSubsets = lib.lookupFunction<_CSubsets, _DSubsets>('vs_index_search_subsets');
    scoreAll = lib.lookupFunction<_CScoreAll, _DScoreAll>('vs_index_score_all');
    reset = lib.lookupFunction<_CGetI32, _DGetI32>('vs_index_reset');
    finalizer = ffi.NativeFinalizer(lib.lookup<ffi.NativeFunction<_CDestroy>>('vs_index_destroy').cast());
  }
  late final _DCreate create;
  late final _DDestroy destroy;
  late final _DAdd add;
  late final _DSearch search;
  late final _DRange range;
  late final _DRangeFree rangeFree;
  late final _DRemove remove;
  late final _DNtotal ntotal;
  late final _DRecon reconstruct;
  late final _DErr lastError;
  late final _DJoin selfJoin;
  late final _DPairsFree pairsFree;
  late final _DKmeans kmeansStep;
  late final _DLoad loadFlat;
  late final _DNtotal indexD;
  late final _DGetI32 indexMetric;
  late final _DSubsets searchSubsets;
  late final _DScoreAll scoreAll;
  late final _DGetI32 reset;
  late final ffi.NativeFinalizer finalizer;

  /// Status -> the exception the reference throws for the same condition.
  void check(int rc) {
    if (rc == _vsOk) return;
    final msg = lastError().toDartString();
    if (rc == _vsInvalid) throw ArgumentError(msg);
    if (rc == _vsUnsupported) throw UnsupportedError(msg);
    throw StateError('libvs_hip: $msg (status $rc)');
  }
}

final _vs = _Vs();

/// One Lloyd iteration's results (kmeans.dart:91-140).
class KmeansStepResult {
  KmeansStepResult(this.assignments, this.centroids, this.counts, this.objective);
  final Int32List assignments;
  final List<Float32List> centroids;
  final Int32List counts;
  final double objective;
}

/// One near-duplicate pair of [GpuIndexFlat.selfJoin]: i < j.
typedef JoinPair = ({int i, int j, double score});

/// Brute-force exact flat index resident on one MI355X.
class GpuIndexFlat extends Index implements ffi.Finalizable {
  GpuIndexFlat._(int d, Metric metric, {int device = 0, bool f32Storage = false})
      : super(d, metric) {
    final out = calloc<ffi.Pointer<ffi.Void>>();
    try {
      _vs.check(_vs.create(device, d, metric == Metric.l2 ? 0 : 1,
          f32Storage ? _storageF32 : _storageAuto, out));
      _h = out.value;
    } finally {
      calloc.free(out);
    }
    _vs.finalizer.attach(this, _h.cast(), detach: this);
  }

  GpuIndexFlat._adopt(ffi.Pointer<ffi.Void> h, int d, Metric metric) : super(d, metric) {
    _h = h;
    _vs.finalizer.attach(this, _h.cast(), detach: this);
  }

  /// gpu_index_flat.dart:47.  `f32Storage`: keep fp32 rows always (the
  /// points of [kmeansStep]); the default stores rows as bf16 while that is
  /// lossless and widens to fp32 at the first row that is not.
  factory GpuIndexFlat.l2(int d, {bool f32Storage = false}) =>
      GpuIndexFlat._(d, Metric.l2, f32Storage: f32Storage);

  /// gpu_index_flat.dart:50.
  factory GpuIndexFlat.ip(int d, {bool f32Storage = false}) =>
      GpuIndexFlat._(d, Metric.innerProduct, f32Storage: f32Storage);

  /// readIndex (FAISDART IndexFlat, index_io.dart:8-26) or readFaissIndex
  /// (IxF2 / IxFI, faiss_io.dart:1690-1716) of a flat index file, with its
  /// rows streamed straight into HBM.  Malformed files throw ArgumentError
  /// with the reference's FormatException text.
  static GpuIndexFlat load(String path, {int device = 0}) {
    final out = calloc<ffi.Pointer<ffi.Void>>();
    final trained = calloc<ffi.Int32>();
    final p = path.toNativeUtf8();
    try {
      _vs.check(_vs.loadFlat(device, p, _storageAuto, out, trained));
      final h = out.value;
      final g = GpuIndexFlat._adopt(
          h, _vs.indexD(h), _vs.indexMetric(h) == 0 ? Metric.l2 : Metric.innerProduct);
      g.isTrained = trained.value != 0;
      return g;
    } finally {
      calloc.free(out);
      calloc.free(trained);
      calloc.free(p);
    }
  }

  /// gpu_index_flat.dart:57: copies an existing IndexFlat's vectors to HBM once.
  factory GpuIndexFlat.wrap(IndexFlat src) {
    final g = GpuIndexFlat._(src.d, src.metric);
    if (src.ntotal > 0) {
      g.add(List<Float32List>.generate(src.ntotal, (i) => src.reconstruct(i)));
    }
    g.isTrained = src.isTrained;
    return g;
  }

  late ffi.Pointer<ffi.Void> _hd;
  bool _disposed = false;

  /// The native handle; a call after [dispose] throws StateError instead of
  /// reaching freed memory.
  ffi.Pointer<ffi.Void> get _h {
    if (_disposed) throw StateError('GpuIndexFlat used after dispose()');
    return _hd;
  }

  set _h(ffi.Pointer<ffi.Void> h) => _hd = h;

  @override
  int get ntotal => _vs.ntotal(_h);
  @override
  set ntotal(int _) {}

  /// gpu_index_flat.dart:85 returns the live CPU IndexFlat the reference
  /// class wraps.  The vectors here live only in HBM, so this returns a
  /// CPU IndexFlat rebuilt from them: a snapshot (later adds to either side
  /// do not reach the other).
  IndexFlat get backing {
    final flat = IndexFlat(d, metric);
    final n = ntotal;
    if (n > 0) {
      final p = calloc<ffi.Float>(n * d);
      try {
        _vs.check(_vs.reconstruct(_h, 0, n, p));
        final v = p.asTypedList(n * d);
        flat.add(List<Float32List>.generate(
            n, (i) => Float32List.fromList(v.sublist(i * d, (i + 1) * d))));
      } finally {
        calloc.free(p);
      }
    }
    flat.isTrained = isTrained;
    return flat;
  }

  /// Vectors are resident after add(); kept for API parity.
  void warmup() {}

  /// Releases the device memory now instead of at finalization.  A second
  /// call does nothing; any other call afterwards throws StateError.
  void dispose() {
    if (_disposed) return;
    _vs.finalizer.detach(this);
    _vs.destroy(_hd);
    _disposed = true;
  }

  ffi.Pointer<ffi.Float> _pack(List<Float32List> rows) {
    final p = calloc<ffi.Float>(rows.length * d);
    final view = p.asTypedList(rows.length * d);
    for (var i = 0; i < rows.length; i++) {
      if (rows[i].length != d) {
        calloc.free(p);
        throw ArgumentError('vector $i has length ${rows[i].length}, expected $d');
      }
      view.setRange(i * d, (i + 1) * d, rows[i]);
    }
    return p;
  }

  @override
  void add(List<Float32List> xs) {
    if (xs.isEmpty) return;
    final p = _pack(xs);
    try {
      _vs.check(_vs.add(_h, p.cast(), _dtypeF32, xs.length));
    } finally {
      calloc.free(p);
    }
  }

  Float32List reconstruct(int id) {
    final p = calloc<ffi.Float>(d);
    try {
      final rc = _vs.reconstruct(_h, id, 1, p);
      if (rc == _vsInvalid) throw RangeError('id $id out of range [0, $ntotal)');
      _vs.check(rc);
      return Float32List.fromList(p.asTypedList(d));
    } finally {
      calloc.free(p);
    }
  }

  @override
  SearchResult search(List<Float32List> queries, int k) {
    final nq = queries.length;
    if (nq == 0) return SearchResult(List<Float32List>.empty(), List<Int32List>.empty());
    final q = _pack(queries);
    final dOut = calloc<ffi.Float>(nq * k);
    final iOut = calloc<ffi.Int32>(nq * k);
    try {
      _vs.check(_vs.search(_h, q.cast(), _dtypeF32, nq, k, dOut, iOut));
      final dv = dOut.asTypedList(nq * k);
      final iv = iOut.asTypedList(nq * k);
      return SearchResult(
        List<Float32List>.generate(nq, (r) => Float32List.fromList(dv.sublist(r * k, (r + 1) * k))),
        List<Int32List>.generate(nq, (r) => Int32List.fromList(iv.sublist(r * k, (r + 1) * k))),
      );
    } finally {
      calloc.free(q);
      calloc.free(dOut);
      calloc.free(iOut);
    }
  }

  @override
  RangeSearchResult rangeSearch(List<Float32List> queries, double radius) {
    final nq = queries.length;
    final q = nq == 0 ? ffi.nullptr.cast<ffi.Float>() : _pack(queries);
    final out = calloc<ffi.Pointer<_RangeC>>();
    try {
      _vs.check(_vs.range(_h, q.cast(), _dtypeF32, nq, radius, out));
      final r = out.value.ref;
      final total = r.lims[nq];
      final limits = Int32List(nq + 1);
      for (var i = 0; i <= nq; i++) {
        limits[i] = r.lims[i];
      }
      final res = RangeSearchResult(limits, Float32List.fromList(r.d.asTypedList(total)),
          Int32List.fromList(r.i.asTypedList(total)));
      _vs.rangeFree(out.value);
      return res;
    } finally {
      if (nq > 0) calloc.free(q);
      calloc.free(out);
    }
  }

  /// Every pair i < j of stored vectors with dot >= threshold (IP) or
  /// squared distance <= threshold (L2), tested on the fp64 score and sorted
  /// by (i, j): the pair list vector_dedup_demo.dart:115-129 builds from
  /// rangeSearch(all, threshold).
  List<JoinPair> selfJoin(double threshold) {
    final out = calloc<ffi.Pointer<_PairsC>>();
    try {
      _vs.check(_vs.selfJoin(_h, threshold, out));
      final r = out.value.ref;
      final pairs = List<JoinPair>.generate(
          r.npairs, (t) => (i: r.i[t], j: r.j[t], score: r.s[t].toDouble()));
      _vs.pairsFree(out.value);
      return pairs;
    } finally {
      calloc.free(out);
    }
  }

  /// One Lloyd iteration of Kmeans.train (kmeans.dart:91-140) with this
  /// index's vectors as the points (create it with `f32Storage: true`):
  /// strict-'<' argmin over the fp64 distances, the fp64 objective in point
  /// order, fp32 running sums in point order times fp64 1/count, and clusters
  /// below minPointsPerCentroid copied from the largest one plus
  /// (u - 0.5) * 1e-4 with u taken in order from `jitter` (the values the
  /// reference draws from its Random).
  KmeansStepResult kmeansStep(List<Float32List> centroids,
      {int minPointsPerCentroid = 1, Float64List? jitter}) {
    final k = centroids.length;
    final n = ntotal;
    final cin = _pack(centroids);
    final ju = calloc<ffi.Double>(jitter == null ? 1 : jitter.length);
    final assign = calloc<ffi.Int32>(n == 0 ? 1 : n);
    final cout = calloc<ffi.Float>(k * d);
    final counts = calloc<ffi.Int32>(k);
    final obj = calloc<ffi.Double>();
    try {
      if (jitter != null) ju.asTypedList(jitter.length).setAll(0, jitter);
      _vs.check(_vs.kmeansStep(_h, cin, k, minPointsPerCentroid, ju, jitter?.length ?? 0, assign,
          cout, counts, obj));
      final cv = cout.asTypedList(k * d);
      return KmeansStepResult(
          Int32List.fromList(assign.asTypedList(n)),
          List<Float32List>.generate(k, (c) => Float32List.fromList(cv.sublist(c * d, (c + 1) * d))),
          Int32List.fromList(counts.asTypedList(k)),
          obj.value);
    } finally {
      calloc.free(cin);
      calloc.free(ju);
      calloc.free(assign);
      calloc.free(cout);
      calloc.free(counts);
      calloc.free(obj);
    }
  }

  /// Exact top-k of each query over subsets of the stored rows (the fine
  /// scan of IndexIVFFlat.search, index_ivf_flat.dart:131-170): query i
  /// scans ids[segOff[i * nseg + s] .. + segLen[i * nseg + s]) for s < nseg;
  /// fp64 scores in dimension order, the k best by (fp32 score, id), -1 /
  /// worst-score sentinels when fewer rows were scanned; any k.
  SearchResult searchSubsets(List<Float32List> queries, int k, Int32List ids, Int64List segOff,
      Int64List segLen, int nseg) {
    final nq = queries.length;
    if (nq == 0) return SearchResult(List<Float32List>.empty(), List<Int32List>.empty());
    if (segOff.length != nq * nseg || segLen.length != nq * nseg) {
      throw ArgumentError('segOff / segLen must hold nq * nseg = ${nq * nseg} entries');
    }
    final q = _pack(queries);
    final pIds = calloc<ffi.Int32>(ids.isEmpty ? 1 : ids.length);
    final pOff = calloc<ffi.Int64>(segOff.isEmpty ? 1 : segOff.length);
    final pLen = calloc<ffi.Int64>(segLen.isEmpty ? 1 : segLen.length);
    final dOut = calloc<ffi.Float>(nq * k);
    final iOut = calloc<ffi.Int32>(nq * k);
    try {
      pIds.asTypedList(ids.length).setAll(0, ids);
      pOff.asTypedList(segOff.length).setAll(0, segOff);
      pLen.asTypedList(segLen.length).setAll(0, segLen);
      _vs.check(_vs.searchSubsets(
          _h, q.cast(), _dtypeF32, nq, k, pIds, ids.length, pOff, pLen, nseg, dOut, iOut));
      final dv = dOut.asTypedList(nq * k);
      final iv = iOut.asTypedList(nq * k);
      return SearchResult(
        List<Float32List>.generate(nq, (r) => Float32List.fromList(dv.sublist(r * k, (r + 1) * k))),
        List<Int32List>.generate(nq, (r) => Int32List.fromList(iv.sublist(r * k, (r + 1) * k))),
      );
    } finally {
      calloc.free(q);
      calloc.free(pIds);
      calloc.free(pOff);
      calloc.free(pLen);
      calloc.free(dOut);
      calloc.free(iOut);
    }
  }

  /// fp32 of the exact fp64 score (l2sq / dot, index.dart:181-200) of every
  /// stored row against q: the closestSq refresh of k-means++
  /// (kmeans.dart:53-84).
  Float32List scoreAll(Float32List q) {
    if (q.length != d) throw ArgumentError('query has length ${q.length}, expected $d');
    final n = ntotal;
    final pq = calloc<ffi.Float>(d);
    final out = calloc<ffi.Float>(n == 0 ? 1 : n);
    try {
      pq.asTypedList(d).setAll(0, q);
      _vs.check(_vs.scoreAll(_h, pq, out));
      return Float32List.fromList(out.asTypedList(n));
    } finally {
      calloc.free(pq);
      calloc.free(out);
    }
  }

  @override
  int removeIds(Set<int> ids) {
    if (ids.isEmpty) return 0;
    final p = calloc<ffi.Int64>(ids.length);
    final removed = calloc<ffi.Int64>();
    try {
      var j = 0;
      for (final id in ids) {
        p[j++] = id;
      }
      _vs.check(_vs.remove(_h, p, ids.length, removed));
      return removed.value;
    } finally {
      calloc.free(p);
      calloc.free(removed);
    }
  }
}

/// Kmeans (kmeans.dart:26-150) with the distance work on the GPU: the
/// k-means++ seeding refreshes closestSq with [GpuIndexFlat.scoreAll] (fp32
/// of the fp64 squared distance, the value `_l2sq` stores), and every Lloyd
/// iteration is one [GpuIndexFlat.kmeansStep] (the assignment and update in
/// the reference's arithmetic).  The same `math.Random(seed)` drives the
/// picks and the empty-cluster jitter in the reference's order: the GPU step
/// copies the largest cluster into an empty one with zero jitter (u = 0.5),
/// and the jitter is drawn and added here, centroid by centroid, exactly as
/// kmeans.dart:127-139 does, so results equal the reference's bit for bit.
class GpuKmeans {
  GpuKmeans({
    required this.d,
    required this.k,
    this.niter = 20,
    this.seed = 1234,
    this.minPointsPerCentroid = 1,
    this.verbose = false,
    this.device = 0,
  });

  final int d;
  final int k;
  final int niter;
  final int seed;
  final int minPointsPerCentroid;
  final bool verbose;
  final int device;

  KmeansResult train(List<Float32List> xs) {
    final n = xs.length;
    if (n < k) {
      throw ArgumentError('k-means: need at least k=$k vectors, got $n');
    }
    final rng = math.Random(seed);
    final pts = GpuIndexFlat._(d, Metric.l2, device: device, f32Storage: true);
    try {
      pts.add(xs);
      // ---- k-means++ (kmeans.dart:48-85) ----
      final centroids = List<Float32List>.generate(k, (_) => Float32List(d));
      centroids[0].setAll(0, xs[rng.nextInt(n)]);
      final closestSq = pts.scoreAll(centroids[0]);
      for (var c = 1; c < k; c++) {
        var sum = 0.0;
        for (var i = 0; i < n; i++) {
          sum += closestSq[i];
        }
        if (sum <= 0) {
          centroids[c].setAll(0, xs[rng.nextInt(n)]);
        } else {
          final target = rng.nextDouble() * sum;
          var acc = 0.0;
          var pick = n - 1;
          for (var i = 0; i < n; i++) {
            acc += closestSq[i];
            if (acc >= target) {
              pick = i;
              break;
            }
          }
          centroids[c].setAll(0, xs[pick]);
        }
        // dsq < closestSq[i] on the fp64 value stores fp32(dsq): the fp32
        // minimum of the refreshed values
        final dsq = pts.scoreAll(centroids[c]);
        for (var i = 0; i < n; i++) {
          if (dsq[i] < closestSq[i]) closestSq[i] = dsq[i];
        }
      }
      // ---- Lloyd iterations (kmeans.dart:88-145) ----
      var cen = centroids;
      var assign = Int32List(n);
      var obj = 0.0;
      final neutral = Float64List(k * d)..fillRange(0, k * d, 0.5);
      for (var it = 0; it < niter; it++) {
        final r = pts.kmeansStep(cen,
            minPointsPerCentroid: minPointsPerCentroid, jitter: neutral);
        final next = r.centroids;
        var big = 0;
        for (var cc = 1; cc < k; cc++) {
          if (r.counts[cc] > r.counts[big]) big = cc;
        }
        for (var c = 0; c < k; c++) {
          if (r.counts[c] >= minPointsPerCentroid) continue;
          // the largest cluster's centroid: its new value when it precedes
          // c (already written, jitter included if it was empty itself),
          // its old one otherwise
          final src = big < c ? next[big] : cen[big];
          final dst = next[c];
          for (var j = 0; j < d; j++) {
            dst[j] = src[j] + (rng.nextDouble() - 0.5) * 1e-4;
          }
        }
        cen = next;
        assign = r.assignments;
        obj = r.objective;
        if (verbose) {
          print('  k-means iter $it obj=${obj.toStringAsFixed(4)}');
        }
      }
      return KmeansResult(cen, assign, obj);
    } finally {
      pts.dispose();
    }
  }
}

/// IndexIVFFlat (index_ivf_flat.dart:16-230) on the GPU: [GpuKmeans] trains
/// the cells, the coarse quantizer is a [GpuIndexFlat] of the centroids (k =
/// 1 assignment at add, the nprobe closest cells at search), the vectors live
/// in HBM in insertion order with the cells' id lists on the host, and the
/// fine scan over the probed lists is [GpuIndexFlat.searchSubsets].  Results
/// equal the reference's except the order inside exact score ties (lowest id
/// first here, heap history there).
class GpuIndexIVFFlat extends Index implements ffi.Finalizable {
  GpuIndexIVFFlat({
    required int d,
    required this.nlist,
    Metric metric = Metric.l2,
    this.nprobe = 1,
    this.kmeansIters = 20,
    this.seed = 1234,
    this.device = 0,
  })  : quantizer = GpuIndexFlat._(d, metric, device: device, f32Storage: true),
        _store = GpuIndexFlat._(d, metric, device: device, f32Storage: true),
        super(d, metric) {
    isTrained = false;
    _invLists = List<List<int>>.generate(nlist, (_) => <int>[]);
  }

  /// Coarse quantizer holding the nlist k-means centroids.
  final GpuIndexFlat quantizer;
  final GpuIndexFlat _store;
  final int nlist;
  int nprobe;
  final int kmeansIters;
  final int seed;
  final int device;
  late List<List<int>> _invLists;

  @override
  int get ntotal => _store.ntotal;
  @override
  set ntotal(int _) {}

  /// invLists[cell]: ids of the vectors assigned to that cell, in insertion
  /// order (index_ivf_flat.dart:52-55).  Do not mutate.
  List<List<int>> get invLists => _invLists;

  /// The stored vectors, [ntotal * d] (index_ivf_flat.dart:47-48), read back
  /// from HBM.
  Float32List get storage {
    final n = ntotal;
    final p = calloc<ffi.Float>(n == 0 ? 1 : n * d);
    try {
      if (n > 0) _vs.check(_vs.reconstruct(_store._h, 0, n, p));
      return Float32List.fromList(p.asTypedList(n * d));
    } finally {
      calloc.free(p);
    }
  }

  /// faiss_io.dart's rehydration hook (index_ivf_flat.dart:60-81): the
  /// vectors go to HBM, the lists replace the current ones.
  void ioSetStorageAndInvLists(Float32List newStorage, List<List<int>> newInvLists, int newNtotal) {
    if (newStorage.length != newNtotal * d) {
      throw ArgumentError('ioSetStorageAndInvLists: storage length ${newStorage.length} '
          '!= ntotal*d = ${newNtotal * d}');
    }
    if (newInvLists.length != nlist) {
      throw ArgumentError(
          'ioSetStorageAndInvLists: got ${newInvLists.length} lists, expected nlist=$nlist');
    }
    _vs.check(_vs.reset(_store._h));
    _store.add(List<Float32List>.generate(
        newNtotal, (i) => Float32List.sublistView(newStorage, i * d, (i + 1) * d)));
    _invLists = newInvLists;
  }

  /// Releases both indexes' device memory.
  void dispose() {
    quantizer.dispose();
    _store.dispose();
  }

  @override
  void train(List<Float32List> xs) {
    if (xs.length < nlist) {
      throw ArgumentError('IndexIVFFlat.train: need >= nlist=$nlist vectors, got ${xs.length}');
    }
    final res = GpuKmeans(d: d, k: nlist, niter: kmeansIters, seed: seed, device: device).train(xs);
    quantizer.add(res.centroids);
    isTrained = true;
  }

  @override
  void add(List<Float32List> xs) {
    if (!isTrained) throw StateError('IndexIVFFlat.add called before train()');
    if (xs.isEmpty) return;
    final assign = quantizer.search(xs, 1);
    final base = ntotal;
    _store.add(xs);
    for (var i = 0; i < xs.length; i++) {
      _invLists[assign.ids[i][0]].add(base + i);
    }
  }

  /// The probed cells' lists as one id array with per-(query, probe)
  /// segments (an unused probe, id -1, is an empty segment).
  (Int32List, Int64List, Int64List) _segments(List<Int32List> probes) {
    final starts = Int64List(nlist + 1);
    for (var c = 0; c < nlist; c++) {
      starts[c + 1] = starts[c] + _invLists[c].length;
    }
    final ids = Int32List(starts[nlist]);
    for (var c = 0; c < nlist; c++) {
      ids.setAll(starts[c], _invLists[c]);
    }
    final nq = probes.length;
    final off = Int64List(nq * nprobe), len = Int64List(nq * nprobe);
    for (var qi = 0; qi < nq; qi++) {
      for (var p = 0; p < nprobe; p++) {
        final cell = probes[qi][p];
        if (cell < 0) continue;
        off[qi * nprobe + p] = starts[cell];
        len[qi * nprobe + p] = starts[cell + 1] - starts[cell];
      }
    }
    return (ids, off, len);
  }

  @override
  SearchResult search(List<Float32List> queries, int k) {
    if (!isTrained) throw StateError('IndexIVFFlat.search before train()');
    if (queries.isEmpty) return SearchResult(List<Float32List>.empty(), List<Int32List>.empty());
    final coarse = quantizer.search(queries, nprobe);
    final (ids, off, len) = _segments(coarse.ids);
    return _store.searchSubsets(queries, k, ids, off, len, nprobe);
  }

  /// index_ivf_flat.dart:173-230: every vector of a probed cell with dist
  /// <= radius (L2) or dot >= radius (IP), in probe order then list order.
  /// The fp64 test runs on the GPU over all stored vectors
  /// ([GpuIndexFlat.rangeSearch]); the hits outside the query's probed
  /// cells are dropped and the rest ordered as the reference emits them.
  @override
  RangeSearchResult rangeSearch(List<Float32List> queries, double radius) {
    if (!isTrained) throw StateError('IndexIVFFlat.rangeSearch before train()');
    final nq = queries.length;
    final all = _store.rangeSearch(queries, radius);
    final coarse = quantizer.search(queries, nprobe);
    final n = ntotal;
    final cellOf = Int32List(n), posOf = Int32List(n);
    for (var c = 0; c < nlist; c++) {
      final l = _invLists[c];
      for (var t = 0; t < l.length; t++) {
        cellOf[l[t]] = c;
        posOf[l[t]] = t;
      }
    }
    final limits = Int32List(nq + 1);
    final dist = <double>[], ids = <int>[];
    final rank = Int32List(nlist);
    for (var qi = 0; qi < nq; qi++) {
      rank.fillRange(0, nlist, -1);
      final probes = coarse.ids[qi];
      for (var p = 0; p < probes.length; p++) {
        if (probes[p] >= 0 && rank[probes[p]] < 0) rank[probes[p]] = p;
      }
      final hits = <int>[];
      for (var t = all.limits[qi]; t < all.limits[qi + 1]; t++) {
        if (rank[cellOf[all.ids[t]]] >= 0) hits.add(t);
      }
      hits.sort((a, b) {
        final ra = rank[cellOf[all.ids[a]]], rb = rank[cellOf[all.ids[b]]];
        return ra != rb ? ra - rb : posOf[all.ids[a]] - posOf[all.ids[b]];
      });
      for (final t in hits) {
        dist.add(all.distances[t]);
        ids.add(all.ids[t]);
      }
      limits[qi + 1] = ids.length;
    }
    return RangeSearchResult(limits, Float32List.fromList(dist), Int32List.fromList(ids));
  }
}

