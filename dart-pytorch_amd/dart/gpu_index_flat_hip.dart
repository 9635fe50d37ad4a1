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
import 'dart:typed_data';

import 'package:ffi/ffi.dart';

import 'index.dart';
import 'index_flat.dart';

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

  late ffi.Pointer<ffi.Void> _h;

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

  /// Releases the device memory now instead of at finalization.
  void dispose() {
    _vs.finalizer.detach(this);
    _vs.destroy(_h);
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
