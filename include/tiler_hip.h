/*
 * tiler_hip.h -- C ABI of the tiler-hip MI355X (gfx950) backend.
 *
 * The reference is a Rust compiler whose backend seams are traits; this ABI is
 * what a thin Rust (or any FFI) shim binds to realize them on MI355X.  Each
 * entry point cites the reference interface it replaces (paths relative to
 * /root/reference/crates/).  Plain pointers and sizes only; no C++ types, no
 * exceptions cross the boundary, and all state lives in a tiler_hip_context
 * (the adapter's `Self`).  One context = one device and one ordered stream,
 * the reference's single-device profile (docs/decisions/0090-...md:152):
 * calls on one context must not overlap from several threads.  Calls that
 * bind the context's device workspace (the tree and multi-pass sums'
 * partials, the split and row-synchronized softmax, the gather record) run
 * on the context's own stream only: given any other stream they refuse with
 * TILER_HIP_REFUSE_UNSUPPORTED before anything is enqueued.
 *
 * Status convention (tiler-runtime/src/adapter.rs:222-231, ADR 0051):
 *   0                 success
 *   negative          Refusal: pre-commit, nothing irreversible happened,
 *                     a fallback route is still permitted
 *   positive          Failure: post-commit, reported and never retried
 *
 * Device pointers are plain device addresses (hipMalloc'd or from
 * tiler_hip_buffer_alloc).  `stream` arguments take a hipStream_t; NULL means
 * the context's own stream.  Launch entry points are asynchronous: they
 * enqueue on the stream and return once the launch is accepted.
 */
#ifndef TILER_HIP_H
#define TILER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t tiler_hip_status;

#define TILER_HIP_OK 0
/* Refusals (pre-commit; RuntimeAdapter::Refusal). */
#define TILER_HIP_REFUSE_NO_DEVICE (-1)
#define TILER_HIP_REFUSE_FOREIGN_TARGET (-2)
#define TILER_HIP_REFUSE_INVALID_ARGUMENT (-3)
#define TILER_HIP_REFUSE_MALFORMED_PAYLOAD (-4)
#define TILER_HIP_REFUSE_ABSENT_SYMBOL (-5)
#define TILER_HIP_REFUSE_BINDING_MISMATCH (-6)
#define TILER_HIP_REFUSE_CAPACITY (-7)
#define TILER_HIP_REFUSE_UNSUPPORTED (-8)
#define TILER_HIP_REFUSE_GATHER_INDEX_OUT_OF_BOUNDS (-9)
#define TILER_HIP_REFUSE_UNRECOGNIZED_KEY (-10)
#define TILER_HIP_REFUSE_NOT_PREPARED (-11)
#define TILER_HIP_REFUSE_PAYLOAD_MISMATCH (-12) /* a payload's metadata names another compilation */
/* Failures (post-commit; RuntimeAdapter::Failure). */
#define TILER_HIP_FAIL_ALLOCATION 1
#define TILER_HIP_FAIL_LAUNCH 2
#define TILER_HIP_FAIL_DEVICE 3
#define TILER_HIP_FAIL_GATHER_INDEX_OUT_OF_BOUNDS 4
#define TILER_HIP_FAIL_TRANSFER 5
#define TILER_HIP_FAIL_VALUE_DOMAIN 6 /* a bound value outside its type's domain, found on the device */

typedef struct tiler_hip_context tiler_hip_context;
typedef void *tiler_hip_stream; /* hipStream_t */
typedef void *tiler_hip_event;  /* hipEvent_t */

/* ------------------------------------------------------------------------
 * Target profile (replaces the declare_* rows of
 * tiler-compiler/src/target/builder.rs:97-1171 and the feasibility axes of
 * target/feasibility.rs:241-256 for gfx950).  Device-free.
 */
typedef struct {
    char profile_key[64];           /* "tiler.hip.gfx950.profile-v1" */
    char target_triple[64];         /* "amdgcn-amd-amdhsa--gfx950" */
    uint32_t wavefront_size;        /* 64 */
    uint32_t compute_units;         /* 256 */
    uint32_t xcds;                  /* 8 accelerator complex dies */
    uint32_t simds_per_cu;          /* 4 */
    uint32_t max_threads_per_workgroup;
    uint32_t max_grid_dim[3];
    uint64_t lds_bytes_per_workgroup; /* 163840 */
    uint64_t device_memory_bytes;     /* 288 GB HBM3E */
    uint64_t l2_bytes_per_xcd;
    uint64_t infinity_cache_bytes;    /* 256 MB MALL */
    uint32_t address_bits;            /* 64 */
    uint32_t index_u64;               /* 1: 64-bit indexing admitted */
    uint32_t subgroup_width;          /* 64: SubgroupRealizationSubject width */
    uint32_t f32_subnormals_preserved;/* 1: IEEE f32 denormals kept */
    double hbm_bytes_per_second;      /* 8.0e12 */
    double mfma_bf16_dense_flops;     /* 2.5e15 */
    double mfma_fp8_dense_flops;      /* 5.0e15 */
    double vector_f32_flops;          /* 157.3e12 */
    double vector_f64_flops;          /* 78.6e12 */
    /* The measured cost row (the reference's saturated-parallel-fold-steps,
     * tiler-compiler/src/target/builder.rs:1369; consumed by
     * tiler-compiler/src/measured_cost.rs): the fold steps the device retires
     * at once when saturated, fitted on an MI355X by the work-span sweep of
     * the sum family's three realizations (tiler_amd.calibrate); where and how
     * it was measured is in cost_row_source. */
    uint64_t saturated_parallel_fold_steps;
    char cost_row_source[192];
} tiler_hip_target_profile;

tiler_hip_status tiler_hip_profile_declare(tiler_hip_target_profile *out);

/* ------------------------------------------------------------------------
 * Producer seam (tiler-build/src/plan_artifact.rs:228-363 assemble_plan_artifact
 * closures; tiler-metal-aot/src/driver.rs:61-453 Toolchain).  The gfx950 code
 * object is compiled offline (clang --offload-device-only) and carried in this
 * library; the payload view describes it the way PayloadMetadata/PayloadProvenance do
 * (tiler-artifact/src/codec/payload.rs:228-424).  Device-free.
 */
typedef struct {
    const char *backend;          /* "tiler.hip" */
    const char *representation;   /* "tiler.hip.gfx950.code-object-v1" */
    const char *payload_schema;   /* "tiler.hip.payload.v1" */
    const char *target;           /* "amdgcn-amd-amdhsa--gfx950" */
    const char *toolchain;        /* compiler identity recorded at build */
    const char *flags;            /* compile flags recorded at build */
    const uint8_t *code;          /* code-object bytes (ELF) */
    uint64_t code_bytes;
    uint32_t entry_count;
    const uint8_t *source;        /* the kernel sources compiled: the build's source bundle
                                     (file count, then each path and contents, u64 big-endian
                                     lengths) */
    uint64_t source_bytes;
} tiler_hip_payload_view;

typedef struct {
    const char *symbol;       /* kernel symbol in the code object */
    const char *family;       /* realization family it serves */
    uint32_t buffer_bindings; /* device-buffer arguments, in kernel order */
    uint32_t kernarg_bytes;   /* kernel argument segment size */
} tiler_hip_entry_info;

tiler_hip_status tiler_hip_payload(tiler_hip_payload_view *out);
tiler_hip_status tiler_hip_payload_entry(uint32_t index, tiler_hip_entry_info *out);

/* The payload's compilation subject, PayloadMetadata, in the artifact layer's
 * canonical encoding (tiler-artifact/src/program/codec/payload.rs:477-580).
 * Every field is an input to the compilation:
 *   - source: the source bundle above;
 *   - toolchain, target, family and language;
 *   - compiler version, the ordered compile flags;
 *   - one entry per kernel: key and symbol, and transports 0..buffers-1;
 *   - two target obligations;
 *   - the unversioned-platform tag.
 * Writes up to `capacity` bytes; *required receives the full length (call
 * with out NULL to size it).  TILER_HIP_REFUSE_CAPACITY if it does not fit. */
tiler_hip_status tiler_hip_payload_metadata(uint8_t *out, uint64_t capacity, uint64_t *required);
/* payload_identity (payload.rs:455-461): the governed digest of those bytes
 * under "tiler.artifact-envelope.payload-identity.v1\0" -- the digest a
 * DeclaredPayload states (tiler-build/tests/custom_backend/backend.rs:451-530). */
tiler_hip_status tiler_hip_payload_identity(uint8_t out[32]);
/* The governed content digest (tiler-digest/src/lib.rs:168-240; algorithm tag
 * 0x01, "tiler.digest.sha-256.v1"): FIPS 180-4 SHA-256 of the domain, then
 * each qualifier in order (fixed width by contract), then the byte run. */
tiler_hip_status tiler_hip_digest(const void *domain, uint64_t domain_bytes,
                                  const void *const *qualifiers, const uint64_t *qualifier_bytes,
                                  uint32_t qualifier_count, const void *bytes, uint64_t byte_count,
                                  uint8_t out[32]);

/* ------------------------------------------------------------------------
 * Artifact envelope reader: what a HIP loader reads of a TILERART envelope
 * (envelope format 1.0, canonical encoding 1.0, manifest schema 22.0;
 * tiler-artifact/src/program/codec/encode.rs:29-306, decode.rs:105-437,
 * validate.rs:68-327).  Device-free; every pointer in a result points into
 * the caller's bytes, which must outlive it.
 *
 * tiler_hip_read_envelope checks, refusing with
 * TILER_HIP_REFUSE_MALFORMED_PAYLOAD and the name of the ArtifactCodecError
 * decode.rs reports first (e.g. "BadMagic", "ManifestDigestMismatch",
 * "SectionDigestMismatch { section: 2 }") in `diagnostic`:
 *   - the 69-byte header: magic, format, encoding, digest algorithm 0x01,
 *     total length, budgets, the manifest digest;
 *   - the manifest through the payload table: domain, schema 22.0,
 *     component schemas, routing policy, features (sorted, distinct,
 *     supported), interface entries, providers and payload descriptors (tags,
 *     budgets, governed keys, canonical order);
 *   - the section descriptors at the manifest's end (count = the header's):
 *     purpose, disposition, schema, and each carried payload's references;
 *   - the section stream: ids, lengths, content digests, no trailing bytes;
 *   - providers present, the embedded-payload-code feature iff a payload is
 *     carried, section order, payload sections referenced, and each carried
 *     payload's identity (its PayloadDigest = payload_identity of its
 *     metadata section, which must decode).
 * The expression arena, variants and delivered-realization record are not
 * parsed (the manifest digest covers them); the identity digest is reported
 * as carried, not re-derived.
 */
typedef struct {
    const uint8_t *backend;            uint64_t backend_bytes;
    const uint8_t *representation;     uint64_t representation_bytes;
    uint16_t payload_schema_major, payload_schema_minor;
    const uint8_t *digest;             uint64_t digest_bytes;  /* PayloadDigest */
    const uint8_t *profile_key;        uint64_t profile_key_bytes;
    const uint8_t *profile_descriptor; uint64_t profile_descriptor_bytes;
    uint32_t has_environment;          /* target-environment declaration present */
    uint32_t carried;                  /* 1: metadata and code below are set */
    uint32_t metadata_section, code_section;
    const uint8_t *metadata;           uint64_t metadata_bytes;
    const uint8_t *code;               uint64_t code_bytes;
} tiler_hip_envelope_payload;

typedef struct {
    uint64_t total_bytes, manifest_bytes;
    uint16_t manifest_schema_major, manifest_schema_minor;
    uint32_t section_count;
    uint8_t section_purpose[64];       /* 1 kernel program, 2 payload metadata, 3 payload code */
    uint64_t feature_count, input_count, output_count, provider_count;
    uint32_t payload_count;
    tiler_hip_envelope_payload payloads[16];
    uint8_t identity_digest[32];       /* as carried */
} tiler_hip_envelope;

tiler_hip_status tiler_hip_read_envelope(const void *bytes, uint64_t byte_count,
                                         tiler_hip_envelope *out, char *diagnostic,
                                         uint64_t diagnostic_bytes);

/* One PayloadEntryMapping (codec/payload.rs:589-640): the entry key, the
 * kernel symbol, and its transports (u32 big-endian each). */
typedef struct {
    const uint8_t *key;        uint64_t key_bytes;
    const uint8_t *symbol;     uint64_t symbol_bytes;
    uint32_t transport_count;
    const uint8_t *transports;
} tiler_hip_payload_mapping;

typedef struct {
    const uint8_t *source_representation; uint64_t source_representation_bytes;
    const uint8_t *source;      uint64_t source_bytes;
    const uint8_t *toolchain;   uint64_t toolchain_bytes;
    const uint8_t *target;      uint64_t target_bytes;
    const uint8_t *family;      uint64_t family_bytes;
    const uint8_t *language;    uint64_t language_bytes;
    uint16_t deployment_major, deployment_minor;
    uint32_t unversioned;       /* 1: the PayloadPlatform::Unversioned tag ends the record */
    uint64_t component_count, compile_flag_count, link_flag_count, obligation_count;
    uint64_t entry_count;
} tiler_hip_payload_subject;

/* decode_metadata (codec/payload.rs:589-660) and check_provenance
 * (payload.rs:291-343).  The first `capacity` mappings go to `mappings`
 * (NULL with capacity 0 to count them). */
tiler_hip_status tiler_hip_read_payload_metadata(const void *bytes, uint64_t byte_count,
                                                 tiler_hip_payload_subject *out,
                                                 tiler_hip_payload_mapping *mappings,
                                                 uint32_t capacity, char *diagnostic,
                                                 uint64_t diagnostic_bytes);

/* The producer's correspondence check (tiler-build/src/payload_cache.rs:522-526
 * takes it; the reference's backends spell it at
 * tiler-build/tests/custom_backend/backend.rs:545-574): does a PayloadMetadata
 * record -- a carried or cached payload's -- describe this library's own
 * compilation (tiler_hip_payload_metadata)?  The facts are read in order:
 * "source-representation", "source", "toolchain", "target", "components",
 * "flags", "entries".  TILER_HIP_OK and "" in `fact` when all agree;
 * TILER_HIP_REFUSE_PAYLOAD_MISMATCH with the first disagreeing fact in `fact`;
 * TILER_HIP_REFUSE_MALFORMED_PAYLOAD (and decode.rs's refusal in `fact`) when
 * the record does not decode. */
tiler_hip_status tiler_hip_payload_correspondence(const void *metadata, uint64_t byte_count, char *fact,
                                                  uint64_t fact_bytes);

/* The carried payload this backend executes (the role tiler-metal-aot's
 * loader plays for its own payloads): backend "tiler.hip", representation
 * "tiler.hip.gfx950.code-object-v1", payload schema major 1, and metadata
 * target "amdgcn-amd-amdhsa--gfx950".  TILER_HIP_REFUSE_FOREIGN_TARGET when
 * the envelope carries none; its entries then route through
 * tiler_hip_prepare_entries with the payload's code bytes. */
tiler_hip_status tiler_hip_select_payload(const tiler_hip_envelope *envelope, uint32_t *index,
                                          char *diagnostic, uint64_t diagnostic_bytes);

/* Validates a code object from its own bytes (ADR 0090 item 8;
 * RuntimeAdapter::validate_payload, tiler-runtime/src/adapter.rs:341):
 * an AMDGPU HSA ELF for gfx950 that defines `symbol` and its kernel descriptor
 * `symbol.kd`, whose kernarg segment is `kernarg_bytes` long (0 = unchecked).
 * Device-free. */
tiler_hip_status tiler_hip_validate_payload(const void *code, uint64_t code_bytes,
                                            const char *symbol, uint32_t kernarg_bytes,
                                            char *diagnostic, uint64_t diagnostic_bytes);

/* ------------------------------------------------------------------------
 * Runtime seam: the RuntimeAdapter stages (tiler-runtime/src/adapter.rs:260-511)
 * driven by route_with_adapter (adapter.rs:545-678).
 */
typedef struct {
    int32_t device_ordinal;
    char device_name[64];
    char gcn_arch_name[64]; /* e.g. "gfx950:sramecc+:xnack-" */
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint32_t max_threads_per_workgroup;
    uint64_t lds_bytes_per_workgroup;
    uint64_t global_memory_bytes;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width_bits;
    int32_t runtime_version;
    int32_t driver_version;
} tiler_hip_execution_environment;

/* bind_execution_context (adapter.rs:293): binds device `ordinal`, creates the
 * context's stream and workspace, loads this library's own gfx950 code object,
 * and reports what it observed.  Refuses a device that is not gfx950. */
tiler_hip_status tiler_hip_bind(int32_t ordinal, tiler_hip_context **out,
                                tiler_hip_execution_environment *environment,
                                char *diagnostic, uint64_t diagnostic_bytes);
void tiler_hip_release(tiler_hip_context *ctx);
const char *tiler_hip_last_diagnostic(const tiler_hip_context *ctx);

/* observe_live_device (adapter.rs:363): reports, never decides.  Keys:
 * "wavefront-size", "compute-units", "max-threads-per-workgroup",
 * "lds-bytes-per-workgroup", "global-memory-bytes", "target-is-gfx950",
 * "max-grid-x", "max-grid-y", "max-grid-z", "device-address-bits", and two
 * measured ones (the rows tiler-compiler/src/target/builder.rs:737-775
 * declares as measured): "f32-input-subnormals" and "f32-result-subnormals".
 * Those run a one-lane probe kernel on the context's stream on first query
 * and answer 1 preserve, 2 flush to a zero of the same sign, 3 flush to +0
 * (0: a pattern none of them produces).
 * Unknown keys answer TILER_HIP_REFUSE_UNRECOGNIZED_KEY (fail-closed). */
tiler_hip_status tiler_hip_observe_live_device(tiler_hip_context *ctx, const char *key,
                                               uint64_t *value);

/* Target environment (RuntimeAdapter::target_environment_support and
 * observe_target_environment, tiler-runtime/src/adapter.rs:295-322; the
 * descriptor schema contract, tiler-artifact/src/program/environment.rs:
 * 249-400).  tiler-hip registers exactly one provider schema, so it never
 * answers Unsupported.  Its canonical descriptor is the bound device's code
 * object target, the one fact a gfx950 code object is compatible with:
 *   u32 BE length, then the target ID "amdgcn-amd-amdhsa--gfx950" followed by
 *   its features in the order the target ID grammar fixes (":sramecc+|-"
 *   then ":xnack+|-"), then u32 BE wavefront size (64).
 * A descriptor is canonical iff it is exactly that spelling for some feature
 * values; every other byte run refuses with a reason. */
typedef struct {
    char provider[64];           /* "tiler.hip.target-environment" */
    uint32_t provider_revision;  /* nonzero: 1 */
    uint16_t schema_major, schema_minor; /* 1.0 */
} tiler_hip_target_environment_schema;

/* target_environment_support: fills the registered schema (device-free). */
tiler_hip_status tiler_hip_target_environment_support(tiler_hip_target_environment_schema *out);
/* validate_canonical_descriptor: TILER_HIP_OK for the schema's one canonical
 * spelling, TILER_HIP_REFUSE_INVALID_ARGUMENT naming the first defect. */
tiler_hip_status tiler_hip_validate_target_environment(const void *descriptor, uint64_t bytes,
                                                       char *diagnostic, uint64_t diagnostic_bytes);
/* observe_target_environment: the bound context's canonical descriptor.
 * *observed = 1 and the bytes (up to `capacity`; *required receives the
 * length), or *observed = 0 (TargetEnvironmentObservation::Unavailable) with
 * the reason in `reason` -- still TILER_HIP_OK: it filters claimed cells and
 * is not a context failure.  TILER_HIP_REFUSE_CAPACITY if the bytes do not
 * fit. */
tiler_hip_status tiler_hip_observe_target_environment(tiler_hip_context *ctx, uint8_t *descriptor,
                                                      uint64_t capacity, uint64_t *required,
                                                      uint32_t *observed, char *reason,
                                                      uint64_t reason_bytes);

typedef struct {
    const void *code;      /* code-object bytes (borrowed for the call) */
    uint64_t code_bytes;
    const char *symbol;
} tiler_hip_routed_entry;

/* prepare_entries (adapter.rs:387): loads each entry's code object and
 * resolves its symbol; reversible.  Prepared entries are numbered from
 * *first_index in order. */
tiler_hip_status tiler_hip_prepare_entries(tiler_hip_context *ctx,
                                           const tiler_hip_routed_entry *entries,
                                           uint32_t count, uint32_t *first_index);

/* observe_prepared_entry (adapter.rs:416): keys "max-threads-per-workgroup",
 * "static-lds-bytes", "private-bytes-per-lane", "vgprs". */
tiler_hip_status tiler_hip_observe_prepared_entry(tiler_hip_context *ctx, uint32_t prepared,
                                                  const char *key, uint64_t *value);

typedef struct {
    uint32_t prepared;         /* index from tiler_hip_prepare_entries */
    uint32_t grid[3];          /* workgroups per dimension */
    uint32_t block[3];         /* threads per workgroup per dimension */
    uint32_t dynamic_lds_bytes;
    const void *kernargs;      /* packed kernel argument segment */
    uint32_t kernarg_bytes;
    uint32_t binding_count;    /* buffer bindings patched into kernargs */
    const uint32_t *binding_slots;   /* slot of each binding */
    const uint32_t *binding_offsets; /* byte offset of its pointer in kernargs */
    uint32_t extent_count;     /* live extents patched into kernargs (32-bit fields) */
    const uint32_t *extent_ids;      /* which of the plan's live extents */
    const uint32_t *extent_offsets;  /* byte offset of its field in kernargs */
} tiler_hip_dispatch_entry;

/* One live input-axis extent a realization reads at dispatch
 * (InputExtentParameter, tiler-ir/src/kernel/model.rs:375-390; the
 * LiveContraction topology's contracted trip count, schedule/model.rs:1429-1450):
 * the extent of axis `axis` of input access `access`, which must lie in
 * [minimum, bound] -- `bound` is what the realization's slot sizes hold. */
typedef struct {
    uint32_t access;
    uint32_t axis;
    uint64_t minimum;
    uint64_t bound;
} tiler_hip_live_extent;

typedef struct {
    uint32_t slot_count;
    const uint64_t *slot_bytes;     /* required bytes per storage slot */
    uint32_t entry_count;
    const tiler_hip_dispatch_entry *entries; /* in execution order */
    /* Optional (NULL: none): per slot, host bytes (slot_bytes[i] of them) that
     * tiler_hip_dispatch uploads into the slot before the first entry runs --
     * a realization's CONSTANT slot.  NULL entries are left alone. */
    const void *const *slot_contents;
    /* The live extents' values for this dispatch (NULL with count 0: none),
     * and the range each must lie in (the realization's live_extents, in
     * order): required whenever extent_count > 0.  Both plan_dispatch
     * (refusal) and dispatch (failure, before any entry is launched) check
     * every value against its range. */
    uint32_t extent_count;
    const uint64_t *extents;
    const tiler_hip_live_extent *extent_ranges;
} tiler_hip_dispatch_plan;

/* plan_dispatch (adapter.rs:453): sizes and checks the route against the
 * profile and the prepared entries, acquiring nothing. */
tiler_hip_status tiler_hip_plan_dispatch(tiler_hip_context *ctx,
                                         const tiler_hip_dispatch_plan *plan);
/* allocate_dispatch (adapter.rs:486): post-commit program storage.  Slots
 * whose caller pointer is non-NULL are caller-supplied and not allocated. */
tiler_hip_status tiler_hip_allocate_dispatch(tiler_hip_context *ctx,
                                             const tiler_hip_dispatch_plan *plan,
                                             void **slot_pointers);
/* dispatch (adapter.rs:506): encodes every entry in order on the context
 * stream, submits, and waits for terminal success. */
tiler_hip_status tiler_hip_dispatch(tiler_hip_context *ctx, const tiler_hip_dispatch_plan *plan,
                                    void *const *slot_pointers);
/* The same encoding on `stream` (NULL: the context's) without the wait, for
 * callers that order or capture the work themselves (a HIP graph, a serving
 * loop).  No counterpart in the reference, whose dispatch always waits.  A
 * plan with constant-slot contents refuses to enqueue under graph capture
 * (upload the slot first); a failed entry is reported, but errors the device
 * raises later surface at the caller's own synchronization.  The live
 * extents are checked as tiler_hip_dispatch checks them. */
tiler_hip_status tiler_hip_enqueue_dispatch(tiler_hip_context *ctx, const tiler_hip_dispatch_plan *plan,
                                            void *const *slot_pointers, tiler_hip_stream stream);
/* Releases the storage tiler_hip_allocate_dispatch acquired for the plan. */
tiler_hip_status tiler_hip_release_dispatch(tiler_hip_context *ctx,
                                            const tiler_hip_dispatch_plan *plan,
                                            void **slot_pointers, const void **caller_owned);

/* ------------------------------------------------------------------------
 * Device storage, transfer, stream and timing plumbing.
 */
tiler_hip_status tiler_hip_buffer_alloc(tiler_hip_context *ctx, uint64_t bytes, void **out);
tiler_hip_status tiler_hip_buffer_free(tiler_hip_context *ctx, void *ptr);
tiler_hip_status tiler_hip_upload(tiler_hip_context *ctx, void *device_dst, const void *host_src,
                                  uint64_t bytes);
tiler_hip_status tiler_hip_download(tiler_hip_context *ctx, void *host_dst,
                                    const void *device_src, uint64_t bytes);
/* Writes `value` to `words` 32-bit words with a kernel (never a memset node,
 * so the call may be captured into a graph). */
tiler_hip_status tiler_hip_fill_u32(tiler_hip_context *ctx, void *device_dst, uint32_t value,
                                    uint64_t words, tiler_hip_stream stream);
/* Device-to-device copy of `bytes`, ordered on `stream` (NULL: the context's). */
tiler_hip_status tiler_hip_copy(tiler_hip_context *ctx, void *device_dst, const void *device_src,
                                uint64_t bytes, tiler_hip_stream stream);
tiler_hip_status tiler_hip_synchronize(tiler_hip_context *ctx);
tiler_hip_stream tiler_hip_context_stream(tiler_hip_context *ctx);
tiler_hip_status tiler_hip_event_create(tiler_hip_context *ctx, tiler_hip_event *out);
tiler_hip_status tiler_hip_event_record(tiler_hip_context *ctx, tiler_hip_event ev,
                                        tiler_hip_stream stream);
tiler_hip_status tiler_hip_event_elapsed_ms(tiler_hip_context *ctx, tiler_hip_event start,
                                            tiler_hip_event stop, float *ms);
tiler_hip_status tiler_hip_event_destroy(tiler_hip_context *ctx, tiler_hip_event ev);

/* Graph capture of a launch sequence (hipStreamBeginCapture ... hipGraphInstantiate),
 * for launch-bound loops: every family entry point below may be captured.  The
 * stream must not be the legacy NULL stream; NULL selects the context stream. */
typedef void *tiler_hip_graph;
tiler_hip_status tiler_hip_capture_begin(tiler_hip_context *ctx, tiler_hip_stream stream);
tiler_hip_status tiler_hip_capture_end(tiler_hip_context *ctx, tiler_hip_stream stream,
                                       tiler_hip_graph *out);
tiler_hip_status tiler_hip_graph_launch(tiler_hip_context *ctx, tiler_hip_graph graph,
                                        tiler_hip_stream stream);
tiler_hip_status tiler_hip_graph_destroy(tiler_hip_context *ctx, tiler_hip_graph graph);

/* ------------------------------------------------------------------------
 * Realization families.  Each replaces one ScalarProgram x ReductionTopology
 * cell the planner selects (tiler-ir/src/schedule/model.rs:661-920,
 * 1327-1555) and is checked against the tiler-reference function cited.
 */

/* Sum over the last axis of a dense [rows, extent] f32 tensor
 * (strict-serial-sum-f32@1; tiler-reference/src/evaluate.rs:498-589). */
#define TILER_HIP_SUM_SERIAL 0      /* ReductionTopology::Serial, bit-exact strict_sum; the zero
                                       default, so an unset plan is the strict fold */
#define TILER_HIP_SUM_TREE 1        /* reassociating two-level tree (declared grouping) */
#define TILER_HIP_SUM_MULTIPASS 2   /* ::MultiPass, bit-exact strict_partitioned_sum
                                       (evaluate.rs:788-832) */
#define TILER_HIP_SUM_COOPERATIVE 3 /* ::CooperativeWorkgroup, bit-exact
                                       cooperative_grouped_sum (evaluate.rs:845-1158) */
typedef struct {
    uint32_t topology;
    uint32_t participant_major; /* cooperative layout: 0 RoundMajor, 1 ParticipantMajor */
    uint64_t partitions;        /* multipass */
    uint64_t participants;      /* cooperative (<= 1024) */
    uint64_t per_partition;     /* multipass / cooperative contributors per cell */
    uint64_t rounds;            /* cooperative */
} tiler_hip_sum_plan;

/* The tree's and the multi-pass split's partials live in the context
 * workspace when they fit (256 KiB): such a call takes NULL or the context's
 * own stream, and refuses any other (TILER_HIP_REFUSE_UNSUPPORTED).  Larger
 * partials are allocated on the given stream. */
tiler_hip_status tiler_hip_sum_f32(tiler_hip_context *ctx, const float *x, uint64_t rows,
                                   uint64_t extent, float *out, const tiler_hip_sum_plan *plan,
                                   tiler_hip_stream stream);
/* tiler_hip_sum_f32 without any allocation, for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference: it exists for
 * those callers only.  Same plan, same kernels and the same bits as
 * tiler_hip_sum_f32; the partials (the tree's workgroup partials, the
 * multi-pass split's) live in a static device array of 8 MiB that each GPU
 * holds until the process ends, resolved per device at tiler_hip_bind.  A
 * plan whose partials exceed 8 MiB refuses with TILER_HIP_REFUSE_CAPACITY.
 * Calls on one GPU share that array: calls that overlap (other streams,
 * other contexts of the same device) race. */
tiler_hip_status tiler_hip_sum_f32_noalloc(tiler_hip_context *ctx, const float *x, uint64_t rows,
                                           uint64_t extent, float *out, const tiler_hip_sum_plan *plan,
                                           tiler_hip_stream stream);
/* Workgroups the single-output tree uses for n contributors (its grouping). */
uint32_t tiler_hip_sum_tree_workgroups(const tiler_hip_context *ctx, uint64_t n);

/* RMS normalization over the last axis (rms-norm-f32@1;
 * tiler-reference/src/rms_norm.rs:405-489).  dtype: TILER_HIP_F32 or
 * TILER_HIP_BF16 (binary32 arithmetic on exactly widened operands, one
 * narrowing of y).  weight_broadcast != 0: w is one row of `extent` shared by
 * every row; otherwise w has the input's shape (the reference's form).  Rows
 * up to 2^32 - 1 elements (see tiler_hip_row_grouping for the fold order). */
#define TILER_HIP_F32 0
#define TILER_HIP_BF16 1
tiler_hip_status tiler_hip_rms_norm(tiler_hip_context *ctx, uint32_t dtype, const void *x,
                                    const void *w, int32_t weight_broadcast, uint64_t rows,
                                    uint64_t extent, uint32_t eps_bits, void *y,
                                    tiler_hip_stream stream);

/* Softmax over the last axis with the governed-maximum shift (softmax-f32@1;
 * tiler-reference/src/softmax.rs:200-315).  Rows longer than 8192 elements
 * fold their exponent sum by segments (tiler_hip_row_grouping); rows of more
 * than 4 segments run each segment in a workgroup of its own.  Up to 2
 * workgroups per CU they synchronize through words in the context's
 * workspace (one launch; waits bounded by 200 us, or by the
 * TILER_HIP_ROW_SYNC_WAIT_TICKS environment variable at bind, in 100 MHz
 * ticks, after which a workgroup computes its row's maximum and sum from the
 * row itself); beyond that they run three launches with the segment partials
 * in the workspace (up to 32768 segments; more are allocated on the stream).
 * A call that binds the workspace takes NULL or the context's own stream and
 * refuses any other (TILER_HIP_REFUSE_UNSUPPORTED), so two such calls never
 * overlap. */
tiler_hip_status tiler_hip_softmax_f32(tiler_hip_context *ctx, const float *x, uint64_t rows,
                                       uint64_t extent, float *y, tiler_hip_stream stream);

/* The declared grouping of a row reduction: thread t of a 64*waves-thread
 * group folds the `vec`-element chunks t, t + 64*waves, ... in ascending
 * position, each wave combines its lanes with an xor butterfly (offsets 32 ..
 * 1) and the wave results are added in ascending order.  segment != 0: the
 * row is cut into segments of `segment` elements, each segment is folded so
 * (chunk positions relative to the segment) and the row total is the left
 * fold of the segment results in ascending order.  RMSNorm and softmax rows
 * of up to 8192 elements use one wave (waves 1, segment 0); longer RMSNorm
 * rows one 1024-thread workgroup (waves 16, segment 0); longer softmax rows
 * segments of 8192 (waves 4); the many-row sum uses (4, 4, 0).  The
 * reassociation is the one the kernels perform whichever launch form runs,
 * reported so a planner can record it.  Device-free. */
#define TILER_HIP_ROWS_RMS_NORM 0
#define TILER_HIP_ROWS_SOFTMAX 1
#define TILER_HIP_ROWS_SUM 2
tiler_hip_status tiler_hip_row_grouping(uint32_t family, uint32_t dtype, uint64_t extent,
                                        uint32_t *vec, uint32_t *waves, uint64_t *segment);

/* Pointwise maps (tiler-reference/src/evaluate.rs:448-485; silu.rs:511-533).
 * op: 0 scale-bias y = x*a + b, 1 SiLU, 2 add x + x2, 3 multiply x * x2.
 * x2_broadcast != 0 reads x2 as a rank-0 operand. */
#define TILER_HIP_MAP_SCALE_BIAS 0
#define TILER_HIP_MAP_SILU 1
#define TILER_HIP_MAP_ADD 2
#define TILER_HIP_MAP_MULTIPLY 3
tiler_hip_status tiler_hip_map(tiler_hip_context *ctx, uint32_t op, uint32_t dtype,
                               const void *x, const void *x2, int32_t x2_broadcast, uint64_t n,
                               float a, float b, void *y, tiler_hip_stream stream);

/* One node of a pointwise expression (PointwiseF32Node,
 * tiler-ir/src/schedule/pointwise.rs:74-140; PointwiseBf16Node,
 * pointwise_bf16.rs:114-168).  Operands name earlier nodes (a DAG in
 * topological order).  INPUT: a = access ordinal (the inputs are dense
 * 0..n-1, each named once).  CONSTANT: a = the constant's bits (binary32, or
 * bf16 in the low 16 bits).  ADD, MULTIPLY, DIVIDE: a = lhs, b = rhs.  EXP,
 * RSQRT: a = argument.  bf16 expressions admit INPUT, CONSTANT, ADD and
 * MULTIPLY only. */
#define TILER_HIP_NODE_INPUT 0u
#define TILER_HIP_NODE_CONSTANT 1u
#define TILER_HIP_NODE_ADD 2u
#define TILER_HIP_NODE_MULTIPLY 3u
#define TILER_HIP_NODE_DIVIDE 4u
#define TILER_HIP_NODE_EXP 5u
#define TILER_HIP_NODE_RSQRT 6u
#define TILER_HIP_MAX_EXPRESSION_NODES 4096u /* MAX_POINTWISE_{F32,BF16}_EXPRESSION_NODES */
typedef struct {
    uint32_t op;
    uint32_t a;
    uint32_t b;
} tiler_hip_expression_node;

/* Pointwise expression DAG (ScalarProgram::PointwiseF32 / PointwiseBf16;
 * tiler-ir/src/schedule/pointwise.rs:74-140, pointwise_bf16.rs:114-168):
 * y[i] = root evaluated on inputs[0..I)[i] for i < n, one fused launch.  The
 * DAG is verified as the reference's builder does (operands defined before
 * use, input ordinals dense and each named once, every node reachable from
 * the root, at most TILER_HIP_MAX_EXPRESSION_NODES nodes, at most 16 inputs).
 * dtype TILER_HIP_F32: ADD, MULTIPLY, DIVIDE round once (IEEE binary32),
 * EXP and RSQRT are correctly rounded, every node's result is canonicalized,
 * and the subnormal modes (TILER_HIP_SUBNORMALS_*, 0: preserve) apply at
 * each node's operands and result (tiler-reference/src/conformance.rs:498-521).
 * dtype TILER_HIP_BF16: bf16 storage, INPUT/CONSTANT/ADD/MULTIPLY, each node
 * rounded once to bf16 (ADR 0091), preserve only.  The register program is
 * uploaded on a call's first use (so a graph may capture only programs the
 * context has already run). */
tiler_hip_status tiler_hip_expression(tiler_hip_context *ctx, uint32_t dtype,
                                      const tiler_hip_expression_node *nodes, uint32_t node_count,
                                      uint32_t root, const void *const *inputs, uint64_t n, void *y,
                                      uint32_t input_subnormals, uint32_t result_subnormals,
                                      tiler_hip_stream stream);

/* Serial fold of a dense row-major f32 tensor (dims[0..rank), rank <= 8)
 * over the axes set in reduced_mask, one output per kept coordinate (kept
 * axes in order): TILER_HIP_FOLD_* (see PROGRAM_FOLD below; scale and bias
 * bits for FMA).  Bit-exact with the reference's strict fold
 * (tiler-reference/src/evaluate.rs:498-589; tiler-ir/src/kernel/lower.rs:
 * 1236-1305, 2485-2500). */
tiler_hip_status tiler_hip_fold_f32(tiler_hip_context *ctx, uint32_t variant, const float *x,
                                    uint32_t rank, const uint64_t *dims, uint64_t reduced_mask,
                                    uint32_t scale_bits, uint32_t bias_bits, float *out,
                                    tiler_hip_stream stream);

/* Reindex move with signed strides (the mirrored reindex,
 * tiler-metal/goldens/structural_mirrored_reindex.metal; structural.rs:75-108):
 * out (row-major over out_dims) element reads source offset
 * base + sum_d coord_d * strides[d].  The smallest and largest offset the
 * geometry reaches must lie in [0, src_elements), else it refuses before any
 * launch.  element_bytes 2 or 4. */
tiler_hip_status tiler_hip_reindex(tiler_hip_context *ctx, const void *src, uint64_t src_elements,
                                   uint32_t rank, const uint64_t *out_dims, const int64_t *strides,
                                   int64_t base, uint32_t element_bytes, void *out,
                                   tiler_hip_stream stream);

/* Broadcast / reindex move (broadcast-f32@2; tiler-reference/src/structural.rs:75-108):
 * out (row-major over out_dims) element reads source offset
 * sum coord_d * src_strides[d] (elements; stride 0 broadcasts). rank <= 8;
 * element_bytes 2 or 4.  The source holds src_elements elements: a geometry
 * whose largest offset falls outside it refuses before any launch. */
tiler_hip_status tiler_hip_broadcast(tiler_hip_context *ctx, const void *src, uint64_t src_elements,
                                     uint32_t rank, const uint64_t *out_dims,
                                     const uint64_t *src_strides, uint32_t element_bytes, void *out,
                                     tiler_hip_stream stream);

/* Gather (gather-f32@1; tiler-reference/src/structural.rs:513-606, bound rule
 * tiler-ir/src/semantic/gather.rs:438-455): source [outer, gathered, inner] of
 * element_bytes elements, 32-bit index (index_signed: int32, else uint32),
 * output [outer, index_count, inner].  Byte moves only.  An out-of-range index
 * is never clamped or wrapped: its run is not written and the lowest offending
 * position is recorded for tiler_hip_gather_status.  The record is the
 * context's: the call takes NULL or the context's own stream and refuses any
 * other (TILER_HIP_REFUSE_UNSUPPORTED). */
tiler_hip_status tiler_hip_gather(tiler_hip_context *ctx, const void *source, uint64_t outer,
                                  uint64_t gathered, uint64_t inner, uint32_t element_bytes,
                                  const uint32_t *index, uint64_t index_count,
                                  int32_t index_signed, void *out, tiler_hip_stream stream);
/* Waits for the stream and reports the gathers since the last call:
 * TILER_HIP_OK, or TILER_HIP_FAIL_GATHER_INDEX_OUT_OF_BOUNDS with the lowest
 * offending position.  Re-arms the record.  NULL or the context's own stream
 * only (TILER_HIP_REFUSE_UNSUPPORTED otherwise). */
tiler_hip_status tiler_hip_gather_status(tiler_hip_context *ctx, tiler_hip_stream stream,
                                         uint64_t *bad_position);
/* Strict per-tensor affine U4 -> f32 dequantization
 * (dequantize-strict-affine; tiler-reference/src/quantization.rs:218-246 and
 * :409-419, ScalarProgram::StrictAffineU4Dequantize, tiler-ir/src/schedule/
 * model.rs:682-696): n codes packed U4 LSB-first in (n + 1) / 2 U8 carriers
 * with a zero tail; y[i] = (code_i - zero_point) * scale as binary32, +0.0
 * where code_i == zero_point.  scale_bits must be a positive normal binary32
 * and zero_point at most 15 (the value contract, quantization.rs:318-370):
 * otherwise TILER_HIP_REFUSE_INVALID_ARGUMENT before anything is enqueued. */
tiler_hip_status tiler_hip_dequantize_u4(tiler_hip_context *ctx, const uint8_t *codes, uint64_t n,
                                        uint32_t scale_bits, uint32_t zero_point, float *y,
                                        tiler_hip_stream stream);

/* Pre-commit form of the same bound rule for host-resident indices:
 * TILER_HIP_REFUSE_GATHER_INDEX_OUT_OF_BOUNDS naming the first position. */
tiler_hip_status tiler_hip_validate_gather_index(const uint32_t *index, uint64_t index_count,
                                                 int32_t index_signed, uint64_t gathered,
                                                 uint64_t *bad_position, int64_t *bad_value);

/* bf16 <-> binary32 conversion, one typed family per direction (ADR 0091
 * decision 2; docs/decisions/0091-...md).  NARROW: binary32 -> bf16, round to
 * nearest even, overflow to a signed infinity at the inclusive midpoint above
 * the largest finite bf16, every NaN -> 0x7fc0, gradual underflow, signed zero
 * kept.  WIDEN: bf16 -> binary32, exact and total (a NaN keeps its payload).
 * n elements; src and dst must not overlap. */
#define TILER_HIP_CONVERT_NARROW_F32_BF16 0
#define TILER_HIP_CONVERT_WIDEN_BF16_F32 1
tiler_hip_status tiler_hip_convert(tiler_hip_context *ctx, uint32_t direction, const void *src,
                                   uint64_t n, void *dst, tiler_hip_stream stream);

/* Contraction td,od->to: C[m, n] = sum_k A[m, k] * B[n, k]
 * (tensor-contraction-f32@1; tiler-reference/src/contraction.rs:297-630). */
/* Strict f32: bit-exact with the reference's fold (first-product seed, no FMA). */
tiler_hip_status tiler_hip_contract_strict_f32(tiler_hip_context *ctx, const float *a,
                                               const float *b, uint64_t m, uint64_t n,
                                               uint64_t k, float *c, tiler_hip_stream stream);
/* Cooperative bf16 on MFMA: bf16 operands, f32 accumulation, optional fused
 * SiLU on the accumulator, one bf16 narrowing of C. */
#define TILER_HIP_EPILOGUE_NONE 0
#define TILER_HIP_EPILOGUE_SILU 1
tiler_hip_status tiler_hip_contract_bf16(tiler_hip_context *ctx, const uint16_t *a,
                                         const uint16_t *b, uint64_t m, uint64_t n, uint64_t k,
                                         uint16_t *c, uint32_t epilogue,
                                         tiler_hip_stream stream);

/* Contraction over any admitted binary index structure (ADR 0087: the
 * reference's ContractionIndexStructure, tiler-ir/src/semantic/contraction.rs:
 * 482-660, evaluated by tiler-reference/src/contraction.rs:346-715).  Each
 * operand is dense row-major with operand_rank[s] axes, axis a labelled
 * operand_indices[s][a] (any uint32) and sized operand_dims[s][a]; the result
 * is dense row-major over output_indices.  Refused (INVALID_ARGUMENT) unless
 * the five structural rules hold (an index repeats within no tuple, every
 * output index names an operand axis, every summed index names an axis of
 * both operands; contraction.rs:804-900), at least one index is summed, the
 * extents of one index agree, and the summed domain is not empty
 * (contraction.rs:420-428).  The contracted set is every operand index absent
 * from the output, ascending by label; its row-major odometer is the
 * contributor sequence.
 *   strict (no PERMITS_REASSOCIATION): the reference fold per output --
 *     seeded at the first product, fl(a*b) and fl(acc + p), no FMA; f32
 *     bit-exact; bf16 operands widened exactly, the f32 fold, optional SiLU,
 *     one bf16 narrowing.
 *   PERMITS_REASSOCIATION, bf16: structures of the form
 *     left [batch.., m, k] x right [batch.., n, k] or [batch.., k, n] ->
 *     out [batch.., m, n] (one summed index; batch axes in any order, each in
 *     either operand or both -- the attention score and value contractions)
 *     run on the MFMA kernels above with batch strides, a right operand
 *     stored [k, n] first transposed into a workspace; other structures take
 *     the strict fold. */
#define TILER_HIP_MAX_CONTRACTION_RANK 8
typedef struct {
    uint32_t operand_rank[2];         /* left, right */
    uint32_t output_rank;
    uint32_t reserved;                /* 0 */
    uint32_t operand_indices[2][8];
    uint32_t output_indices[8];
    uint64_t operand_dims[2][8];
} tiler_hip_contraction_structure;
/* dtype TILER_HIP_F32 (epilogue NONE) or TILER_HIP_BF16; permissions
 * TILER_HIP_PERMITS_*.  The workspace a [k, n] right operand needs is
 * allocated on the stream (refused under graph capture); the strict form's
 * geometry is uploaded once per distinct structure and kept by the context. */
tiler_hip_status tiler_hip_contract(tiler_hip_context *ctx, uint32_t dtype,
                                    const tiler_hip_contraction_structure *structure,
                                    uint32_t epilogue, uint32_t permissions, const void *left,
                                    const void *right, void *out, tiler_hip_stream stream);

/* ------------------------------------------------------------------------
 * Realization recognizer: one scheduled region -> the dispatches that realize
 * it on this library's entry points.  It takes the role of tiler-metal's
 * emit_entry_point (tiler-metal/src/emit.rs:647-840) for a backend whose code
 * is built ahead of time. Inputs:
 *   - the region's ScalarProgram (tiler-ir/src/schedule/model.rs:661-930);
 *   - its ReductionTopology (model.rs:1327-1555);
 *   - its geometry, which the planner's KernelSchedule/LaunchPlan summarizes
 *     (model.rs:1785-1812).
 * The result is exactly the program the family entry point above runs for
 * the same request. It is what the runtime seam executes:
 *   1. tiler_hip_prepare_entries on the payload symbols the entries name;
 *   2. tiler_hip_plan_dispatch;
 *   3. tiler_hip_allocate_dispatch;
 *   4. tiler_hip_dispatch.
 * Device-free: with ctx NULL the declared profile's 256 CUs decide the tile
 * size and the tree grouping; with a context, its device's CUs do.
 */
#define TILER_HIP_PROGRAM_POINTWISE 1   /* ScalarProgram::PointwiseF32 / PointwiseBf16 (model.rs:663, 681) */
#define TILER_HIP_PROGRAM_SERIAL_SUM 2  /* ::StrictSerialSum (model.rs:698) */
#define TILER_HIP_PROGRAM_RMS_NORM 3    /* ::SquaredSerialSumThenEpilogue (model.rs:815) */
#define TILER_HIP_PROGRAM_SOFTMAX 4     /* law StagedSoftmaxF32 (tiler-ir/src/index/law.rs:289) over
                                           ::StrictSerialMaximum (model.rs:920) */
#define TILER_HIP_PROGRAM_CONTRACTION 5 /* ::StrictTensorContraction (model.rs:850) */
#define TILER_HIP_PROGRAM_GATHER 6      /* tiler-reference/src/structural.rs:513-606 */
#define TILER_HIP_PROGRAM_BROADCAST 7   /* tiler-reference/src/structural.rs:75-108 */
#define TILER_HIP_PROGRAM_CONVERT 8     /* the ADR 0091 conversion families; variant: TILER_HIP_CONVERT_* */
#define TILER_HIP_PROGRAM_EXPRESSION 9  /* ::PointwiseF32 / ::PointwiseBf16 expression DAGs (model.rs:663,
                                           681; schedule/pointwise.rs, pointwise_bf16.rs): nodes, root */
#define TILER_HIP_PROGRAM_FOLD 10       /* the serial folds over any reduced axis set (variant:
                                           TILER_HIP_FOLD_*): StrictSerialSum (model.rs:698),
                                           FusedMultiplyAddSerialSum (:709), SquaredSerialSum (:745),
                                           StrictSerialMaximum (:920) */
#define TILER_HIP_PROGRAM_REINDEX 11    /* structural reindex with signed strides (the mirrored reindex,
                                           tiler-metal/goldens/structural_mirrored_reindex.metal) */
#define TILER_HIP_PROGRAM_DEQUANTIZE_U4 12 /* ::StrictAffineU4Dequantize (model.rs:682-696): slots codes,
                                              scale, zero point, y, and a 4-byte scratch slot where the
                                              kernel records the operands' domain verdict (0 in domain,
                                              1 scale, 2 zero point); extents[0] = element count */

/* PROGRAM_FOLD variants.  The input is dense row-major with `rank` dims in
 * extents[]; grouping[0] is the reduced-axis mask (bit d: axis d reduced);
 * the output is the kept axes, dense, in order.  Each output folds its
 * contributors in lexicographic order of the reduced coordinates, seeded at
 * the first contributor (evaluate.rs:548-585); every combine is canonical.
 *   SUM      acc = acc + x                         empty: +0 (empty_identity_bits)
 *   SQUARED  acc = acc + fl(x * x)                 empty: +0
 *   FMA      acc = acc + fl(fl(x * scale) + bias)  scalars {scale, bias}; the
 *            program's `contraction` permission (FusedMultiplyAddSerialSum::
 *            contraction) is not consumed: the two-rounding form is the one
 *            every contract admits                 empty: +0
 *   MAXIMUM  NaN-propagating IEEE maximum with -0 < +0 (softmax.rs:168-186);
 *            order-insensitive, so it spends no reassociation permission;
 *            an empty reduced domain is refused (model.rs:880-906)
 * The sums take the region's topology: SERIAL (any axes), or, under
 * PERMITS_REASSOCIATION and over the trailing axis only, MULTIPASS
 * (grouping[1] partitions of grouping[2]) and COOPERATIVE (grouping[1]
 * participants, grouping[2] contributors per cell, RoundMajor unless
 * TILER_HIP_REGION_PARTICIPANT_MAJOR, the rounds that cover the axis).
 * Under a flushing contract every arithmetic site of the prologue and of
 * each combine applies the declared modes, every fold seeded at its first
 * contributor (evaluate.rs:575-583, 612-832, 845-1158); the maximum takes no
 * mode.  An epilogue is realized serially under the preserving modes only. */
#define TILER_HIP_FOLD_SUM 0u
#define TILER_HIP_FOLD_SQUARED 1u
#define TILER_HIP_FOLD_FMA 2u
#define TILER_HIP_FOLD_MAXIMUM 3u

/* Region flags. */
#define TILER_HIP_REGION_ALIGNED16 1u         /* precondition: every slot's base address is 16-byte aligned */
#define TILER_HIP_REGION_OPERAND_BROADCAST 2u /* pointwise: x2 is one element; rms_norm: w is one row */
#define TILER_HIP_REGION_INDEX_SIGNED 4u      /* gather: int32 indices */
#define TILER_HIP_REGION_PARTICIPANT_MAJOR 8u /* cooperative sum layout */
#define TILER_HIP_REGION_LIVE_EXTENT 16u      /* contraction td,od->to: k is live (LiveContraction), read at
                                                 dispatch as the realization's live extent 0 (input 0, axis 1);
                                                 extents[2] is its bound */

/* The plan's numerical contract as it reaches one region: the permissions
 * its ReductionTopology carries (permits_reassociation, permits_permutation;
 * tiler-ir/src/schedule/model.rs:1330-1340, 1409-1413, 1520-1540) and the two
 * subnormal dimensions of the resolved contract (STRICT_F32,
 * FLUSH_SUBNORMALS_TO_ZERO_F32, REASSOCIATE_F32, FLUSH_AND_REASSOCIATE_F32,
 * STRICT_BF16 ...; tiler-compiler/src/session.rs:1793-1888).  All zero is the
 * strict contract: no regrouping of any fold, subnormals preserved.
 *   - A reassociating realization (the two-level tree sum, the multi-pass and
 *     cooperative splits, the grouped RMSNorm and softmax row folds, the MFMA
 *     contraction) is chosen only under PERMITS_REASSOCIATION.  Without it the
 *     region gets the strict serial fold where this library has one (sum,
 *     RMSNorm, softmax, contraction) and is refused otherwise.  The maximum is
 *     order-insensitive on every binary32 input and spends no permission.
 *   - Subnormal modes: the device preserves binary32 and bf16 subnormals.
 *     A flushing mode is realized where the kernels implement it (pointwise
 *     expressions) and refused before commit everywhere else.  Byte moves
 *     (gather, broadcast) perform no arithmetic and ignore the modes. */
#define TILER_HIP_PERMITS_REASSOCIATION 1u
#define TILER_HIP_PERMITS_PERMUTATION 2u
#define TILER_HIP_SUBNORMALS_PRESERVE 1u       /* 0 reads as PRESERVE */
#define TILER_HIP_SUBNORMALS_FLUSH_SIGN 2u     /* to the zero of the operand's sign */
#define TILER_HIP_SUBNORMALS_FLUSH_POSITIVE 3u /* to +0 */

typedef struct {
    uint32_t program;      /* TILER_HIP_PROGRAM_* */
    uint32_t topology;     /* serial sum: TILER_HIP_SUM_* */
    uint32_t dtype;        /* TILER_HIP_F32 / TILER_HIP_BF16 */
    uint32_t variant;      /* pointwise: TILER_HIP_MAP_*; contraction (bf16): TILER_HIP_EPILOGUE_*;
                              convert: TILER_HIP_CONVERT_*;
                              gather, broadcast: element bytes */
    uint32_t flags;        /* TILER_HIP_REGION_* */
    uint32_t rank;         /* broadcast: output rank (<= 8) */
    uint64_t extents[8];   /* pointwise, convert, expression {n}; sum, rms_norm, softmax {rows, extent};
                              contraction {m, n, k}; gather {outer, gathered, inner, index count};
                              broadcast, reindex: the output dims; fold: the input dims */
    uint64_t strides[8];   /* broadcast: source stride (elements) per output axis;
                              reindex: the same as int64 (two's complement, may be negative) */
    uint64_t grouping[3];  /* multi-pass sum {partitions, per partition};
                              cooperative sum {participants, per partition, rounds};
                              broadcast {source elements}; reindex {source elements, base offset};
                              fold {reduced-axis mask, then the split's or the
                              workgroup's two grouping fields} */
    uint32_t scalars[2];   /* rms_norm {eps bits}; pointwise {a bits, b bits} */
    uint32_t permissions;        /* TILER_HIP_PERMITS_*: the contract's regrouping freedoms */
    uint32_t input_subnormals;   /* TILER_HIP_SUBNORMALS_* (0: preserve) */
    uint32_t result_subnormals;  /* TILER_HIP_SUBNORMALS_* (0: preserve) */
    /* PROGRAM_EXPRESSION: node_count nodes (<= TILER_HIP_MAX_EXPRESSION_NODES)
     * and the root's index; the nodes are read during the call only. */
    uint32_t node_count;
    uint32_t root;
    const tiler_hip_expression_node *nodes;
    /* PROGRAM_CONTRACTION: NULL is td,od->to over extents {m, n, k}; else the
     * index structure (read during the call only), extents unused. */
    const tiler_hip_contraction_structure *structure;
    /* TILER_HIP_FORM_*: 0 lets the library choose the realization; a proposal
     * of tiler_hip_propose names the form it offered.  A form the program
     * does not have, or one the request's shape does not admit, refuses. */
    uint32_t form;
    uint32_t reserved;     /* 0 */
} tiler_hip_region;

/* Forms a region may name (tiler_hip_region.form).  The contraction forms
 * apply to td,od->to bf16 under PERMITS_REASSOCIATION; the softmax forms to
 * rows of more than four 8192-element segments under PERMITS_REASSOCIATION. */
#define TILER_HIP_FORM_AUTO 0u
#define TILER_HIP_FORM_CONTRACT_SKINNY 1u     /* m <= 64: B streamed once, 16 columns per workgroup */
#define TILER_HIP_FORM_CONTRACT_STAGED_256 2u /* 256x256 tiles, 16 waves, LDS-DMA double buffer */
#define TILER_HIP_FORM_CONTRACT_STAGED_128 3u /* 128x128 tiles, 4 waves, the same schedule */
#define TILER_HIP_FORM_CONTRACT_GENERAL_128 4u /* register-staged 128x128 tiles, any n and k */
#define TILER_HIP_FORM_SOFTMAX_SPLIT 5u       /* three launches over segment partials in scratch */
#define TILER_HIP_FORM_SOFTMAX_ROW_SYNC 6u    /* one row-synchronized launch (at most two workgroups per CU) */

/* Storage slot roles.  Slot order per program:
 *   expression  the inputs in access order, y, program (a constant slot)
 *   fold        x, out
 *   reindex     src, out
 *   pointwise   x, [x2,] y       (x2 only for ADD and MULTIPLY)
 *   serial sum  x, out, [partials: scratch]
 *   rms_norm    x, w, y
 *   softmax     x, y
 *   contraction a [m, k], b [n, k], c [m, n]; with a structure: left, right,
 *               out, [the transposed right operand: scratch]
 *   gather      source, index, out, record (scratch: u64, all ones unless an index was
 *               out of range; then the lowest such position).  The program arms the
 *               record itself; validate host indices first (tiler_hip_validate_gather_index).
 *   broadcast   src, out
 *   convert     src, dst */
#define TILER_HIP_SLOT_INPUT 0
#define TILER_HIP_SLOT_OUTPUT 1
#define TILER_HIP_SLOT_SCRATCH 2
#define TILER_HIP_SLOT_CONSTANT 3 /* read-only; the route uploads the realization's `constant`
                                     bytes into it before the first dispatch */
#define TILER_HIP_REALIZATION_CONSTANT_BYTES 49152u /* 4096 nodes of 12 bytes */

typedef struct {
    uint32_t entry;             /* payload entry index (tiler_hip_payload_entry names it) */
    uint32_t grid[3];           /* workgroups */
    uint32_t block[3];          /* threads per workgroup */
    uint32_t kernarg_bytes;
    uint8_t kernargs[256];      /* argument segment; pointer fields are bound at dispatch */
    uint32_t binding_count;
    uint32_t binding_slots[18];
    uint32_t binding_offsets[18];
    uint32_t extent_count;      /* live extents this entry reads (tiler_hip_dispatch_entry) */
    uint32_t extent_ids[2];
    uint32_t extent_offsets[2];
} tiler_hip_realized_entry;

typedef struct {
    uint32_t slot_count;
    uint32_t slot_roles[18];    /* TILER_HIP_SLOT_* */
    uint64_t slot_bytes[18];
    uint32_t slot_alignment;    /* precondition on every slot base: 16 with ALIGNED16, else 1 */
    uint32_t entry_count;       /* 0: zero work, nothing to dispatch */
    tiler_hip_realized_entry entries[4]; /* in execution order */
    uint32_t constant_slot;     /* the CONSTANT slot (slot_count when there is none) */
    uint32_t constant_bytes;    /* its contents: constant[0 .. constant_bytes) */
    uint8_t constant[TILER_HIP_REALIZATION_CONSTANT_BYTES];
    uint32_t live_extent_count; /* REGION_LIVE_EXTENT: the extents the dispatch supplies, by id */
    tiler_hip_live_extent live_extents[2];
} tiler_hip_realization;

/* Refuses (pre-commit, typed) what the family entry point would refuse for
 * the same request, plus TILER_HIP_REFUSE_UNSUPPORTED for a program or
 * dtype this library does not realize. */
tiler_hip_status tiler_hip_realize(const tiler_hip_context *ctx, const tiler_hip_region *region,
                                   tiler_hip_realization *out, char *diagnostic,
                                   uint64_t diagnostic_bytes);

/* ------------------------------------------------------------------------
 * Physical-implementation provider (PhysicalImplementationProvider::propose,
 * tiler-compiler/src/frontier.rs:1507-1527; ProviderOffer :1466-1495).
 * Everything this library can run for one region, so that its gfx950 tile
 * widths, workgroup sizes and dispatch counts are visible to a planner: every
 * strategy it has for the region's program, each either proposed -- with the
 * region to realize for it, its launch geometry and its structural cost -- or
 * declined with the cause the reference's StrategyDeclineCause names
 * (frontier.rs:1311-1384).  An empty offer is not an error.  The offer
 * depends only on its inputs (deterministic, no device access; ctx may be
 * NULL, as for tiler_hip_realize).
 *
 * Strategy keys: the reference's own where the strategy is the reference's
 * ("tiler.region.serial-baseline", "tiler.reduction.multi-pass-split",
 * "tiler.reduction.single-workgroup-tree"; physical.rs:551,3241,3570), and
 * "gfx950." keys for this library's own forms. */
#define TILER_HIP_MAX_PROPOSALS 6
#define TILER_HIP_DECLINE_NUMERICAL_PERMISSION_REFUSED 1u /* subject: the dimension key ("numerics.reassociation") */
#define TILER_HIP_DECLINE_NO_ADMISSIBLE_SHAPE 2u          /* subject: the rule; extent: the extent that admitted none */
#define TILER_HIP_DECLINE_UNREPRESENTABLE 3u              /* subject: the rule (the planner's refusal) */

typedef struct {
    char strategy[64];
    tiler_hip_region region;       /* the request with this strategy's choices (form, topology, grouping):
                                      tiler_hip_realize on it gives exactly this implementation */
    /* PhysicalCostEstimate::structural (frontier.rs:351-400; model tiler.cost.structural.v1) */
    uint32_t dispatch_count;
    uint64_t launched_threads;
    uint64_t temporary_bytes;      /* scratch slots */
    /* The launches, in order: kernel, workgroups (x * y) and threads per workgroup. */
    char symbols[4][48];
    uint64_t workgroups[4];
    uint32_t workgroup_threads[4];
    /* The measured cost row's selector (tiler-compiler/src/measured_cost.rs:60-110;
     * key tiler.cost.measured-fold-steps.v1): sum over stages of max(work, depth * P)
     * with P the profile's saturated_parallel_fold_steps.  Assessed for the
     * sum's strategies, where the row was fitted; 0 elsewhere. */
    uint64_t measured_fold_steps;
} tiler_hip_proposal;

typedef struct {
    char strategy[64];
    uint32_t cause;                /* TILER_HIP_DECLINE_* */
    char subject[64];
    uint64_t extent;
} tiler_hip_declined_strategy;

typedef struct {
    char provider[64];             /* provenance */
    uint32_t proposal_count;
    uint32_t declined_count;
    uint32_t chosen;               /* the proposal tiler_hip_realize picks with form AUTO (its index), or
                                      the measured row's least fold steps among the sum's proposals */
    tiler_hip_proposal proposals[TILER_HIP_MAX_PROPOSALS];
    tiler_hip_declined_strategy declined[TILER_HIP_MAX_PROPOSALS];
} tiler_hip_provider_offer;

/* Refuses only what no strategy could read: a NULL region or offer, an
 * unknown program, a malformed request every strategy refuses the same way
 * (then the diagnostic names it).  A region that names a form is proposed as
 * if it named none. */
tiler_hip_status tiler_hip_propose(const tiler_hip_context *ctx, const tiler_hip_region *region,
                                   tiler_hip_provider_offer *offer, char *diagnostic,
                                   uint64_t diagnostic_bytes);

#ifdef __cplusplus
}
#endif

#endif /* TILER_HIP_H */
