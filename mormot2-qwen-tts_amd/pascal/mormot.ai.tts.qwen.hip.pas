/// the MI355X (gfx950) frame-step engine libq3h, bound for mORMot 2 hosts
// - the C ABI of include/q3h.h, one declaration per entry point, cdecl
// - TQwen3Hip / TQwen3HipContext stand where mormot.ai.tts.qwen.lm.pas uses
// TQwen3Vulkan and its TDecoderContext (lm.pas:351-354, 377, 397)
// - structures go to the library by explicit pointer (PQ3h...), never as
// const records, so the calling convention cannot pass them by value
unit mormot.ai.tts.qwen.hip;

{$ifdef FPC}
  {$mode delphi}
  {$packrecords C}
{$else}
  {$A8}
{$endif}

interface

uses
  SysUtils;

const
  LIBQ3H = 'libq3h.so';

  Q3H_F32 = 0;
  Q3H_Q8_0 = 1;
  Q3H_BF16 = 2;

  Q3H_OK = 0;
  Q3H_E_ARG = -1;
  Q3H_E_HIP = -2;
  Q3H_E_CAPACITY = -3;
  Q3H_E_STATE = -4;
  Q3H_E_NODEV = -5;

  Q3H_NOALLOC_MAX_ROWS = 64;
  Q3H_NOALLOC_SCRATCH_BYTES = 16 shl 20;

type
  PPSingle = ^PSingle;

  /// opaque handles
  q3h_device = pointer;
  q3h_stack = pointer;
  q3h_context = pointer;
  q3h_frame = pointer;
  q3h_text_proj = pointer;
  q3h_codec = pointer;
  Pq3h_context = ^q3h_context;

  /// TDecoderConfig + KvF16 + the numerics of the Q8_0 products
  q3h_stack_config = record
    layers, hidden, heads, kv_heads, head_dim, intermediate: integer;
    rms_eps, rope_theta: single;
    dtype: integer;         // Q3H_F32 or Q3H_Q8_0
    kv_f16: integer;        // K/V cache in half floats (lm.pas:128-130)
    act_q8: integer;        // Q8_0 only: activations quantized per 32-block
    max_positions: integer;
  end;
  Pq3h_stack_config = ^q3h_stack_config;

  /// one layer, host memory, matrices [out][in] row-major in src_dtype
  q3h_layer_weights = record
    wq, wk, wv, wo, wgate, wup, wdown: pointer;
    input_norm, post_norm: PSingle; // [hidden]
    q_norm, k_norm: PSingle;        // [head_dim]
  end;
  Pq3h_layer_weights = ^q3h_layer_weights;

  q3h_weights = record
    src_dtype: integer;             // Q3H_F32, Q3H_Q8_0 (ggml blocks) or Q3H_BF16
    layers: Pq3h_layer_weights;     // [layers]
    final_norm: PSingle;            // [hidden]
  end;
  Pq3h_weights = ^q3h_weights;

  q3h_frame_config = record
    n_streams, talker_head: integer;
    cp_heads: array[0..14] of integer;
    vocab, cp_vocab, groups, eos: integer;
    repetition_penalty: single;
    max_frames, max_positions, use_graph: integer;
  end;
  Pq3h_frame_config = ^q3h_frame_config;

  q3h_sampling = record
    do_sample: integer;
    temperature: single;
    top_k: integer;
    top_p: single;
    sub_do_sample: integer;
    sub_temperature: single;
    sub_top_k: integer;
    sub_top_p: single;
    seed: UInt64;
  end;
  Pq3h_sampling = ^q3h_sampling;

  q3h_text_config = record
    text_vocab, text_hidden, hidden, emb_dtype: integer;
  end;
  Pq3h_text_config = ^q3h_text_config;

  q3h_start_ids = record
    tts_bos, tts_eos, tts_pad, codec_pad, codec_bos: integer;
  end;
  Pq3h_start_ids = ^q3h_start_ids;

  /// the decoder's back part, f32 host arrays in their safetensors layouts
  q3h_codec_res = record
    a1_alpha, a1_beta, c1_w, c1_b, a2_alpha, a2_beta, c2_w, c2_b: PSingle;
  end;
  q3h_codec_block = record
    act_alpha, act_beta, up_w, up_b: PSingle;
    res: array[0..2] of q3h_codec_res;
  end;
  q3h_codec_weights = record
    up_w, up_b, dw_w, dw_b, norm_w, norm_b, pw1_w, pw1_b, pw2_w, pw2_b, gamma:
      array[0..1] of PSingle;
    conv0_w, conv0_b: PSingle;
    block: array[0..3] of q3h_codec_block;
    out_alpha, out_beta, out_w, out_b: PSingle;
  end;
  Pq3h_codec_weights = ^q3h_codec_weights;

{ device: TQwenVulkan (lm.pas:44-62, 202-222) }
function q3h_device_available: integer; cdecl; external LIBQ3H;
function q3h_device_open(ordinal: integer; out dev: q3h_device): integer;
  cdecl; external LIBQ3H;
function q3h_device_name(dev: q3h_device): PAnsiChar; cdecl; external LIBQ3H;
function q3h_device_bytes(dev: q3h_device): Int64; cdecl; external LIBQ3H;
function q3h_device_close(dev: q3h_device): integer; cdecl; external LIBQ3H;
function q3h_last_error: PAnsiChar; cdecl; external LIBQ3H;

{ stack: TQwen3Model.CreateStack + TQwen3Vulkan.Create (lm.pas:174-179, 351) }
function q3h_stack_create(dev: q3h_device; cfg: Pq3h_stack_config;
  w: Pq3h_weights; out s: q3h_stack): integer; cdecl; external LIBQ3H;
function q3h_stack_add_head(s: q3h_stack; w: pointer; rows, src_dtype: integer;
  out index: integer): integer; cdecl; external LIBQ3H;
function q3h_stack_bytes(s: q3h_stack): Int64; cdecl; external LIBQ3H;
function q3h_stack_destroy(s: q3h_stack): integer; cdecl; external LIBQ3H;

{ context: NewContext / TDecoderContext (lm.pas:354, 374-378) }
function q3h_context_create(s: q3h_stack; max_positions: integer;
  out c: q3h_context): integer; cdecl; external LIBQ3H;
function q3h_context_reset(c: q3h_context): integer; cdecl; external LIBQ3H;
function q3h_context_length(c: q3h_context): integer; cdecl; external LIBQ3H;
function q3h_context_destroy(c: q3h_context): integer; cdecl; external LIBQ3H;
function q3h_context_fill_kv(c: q3h_context; k, v: PSingle; len: integer): integer;
  cdecl; external LIBQ3H;
function q3h_context_read_kv(c: q3h_context; layer: integer; k, v: PSingle): integer;
  cdecl; external LIBQ3H;
function q3h_context_time_attention(c: q3h_context; iters: integer;
  out us_per_launch: single; out bytes_per_launch: Int64): integer;
  cdecl; external LIBQ3H;

{ the forward: TQwenLm.Forward (lm.pas:391-408), the head on the device }
function q3h_forward_embeds(c: q3h_context; x: PSingle; rows, head: integer;
  logits, normed_last: PSingle): integer; cdecl; external LIBQ3H;
/// TQwenLm.Forward with its Probe (lm.pas:380-389): layer_out [layers][rows]
// [hidden] receives the raw output of every layer (name.layerN), normed_rows
// [rows][hidden] the final-normed state of every row (name.out)
function q3h_forward_embeds_probe(c: q3h_context; x: PSingle; rows, head: integer;
  logits, normed_last, layer_out, normed_rows: PSingle): integer; cdecl; external LIBQ3H;
/// no counterpart in the reference: q3h_forward_embeds for callers that
// cannot allocate device memory (work buffers in a static device array of
// Q3H_NOALLOC_SCRATCH_BYTES per GPU; rows <= Q3H_NOALLOC_MAX_ROWS)
function q3h_forward_embeds_noalloc(c: q3h_context; x: PSingle; rows, head: integer;
  logits, normed_last: PSingle): integer; cdecl; external LIBQ3H;
function q3h_forward_embeds_batch(ctxs: Pq3h_context; n: integer; x: PSingle;
  heads: PInteger; logits, normed: PSingle): integer; cdecl; external LIBQ3H;

{ the frame step: TQwenTalker.NextFrame on the device (talker.pas:640-681) }
function q3h_frame_create(talker, cp: q3h_stack; cfg: Pq3h_frame_config;
  codec_emb: PSingle; pred_emb: PPSingle; tts_pad: PSingle;
  out f: q3h_frame): integer; cdecl; external LIBQ3H;
function q3h_frame_start(f: q3h_frame; stream: integer; prefill: PSingle;
  rows: integer; trailing: PSingle; trailing_rows: integer): integer;
  cdecl; external LIBQ3H;
/// no counterpart in the reference (batched serving): the starts of n streams
// at once, their prefills overlapping on the device
function q3h_frame_start_batch(f: q3h_frame; n: integer; streams: PInteger;
  prefill: PPSingle; rows: PInteger; trailing: PPSingle;
  trailing_rows: PInteger): integer; cdecl; external LIBQ3H;
function q3h_frame_step(f: q3h_frame; codes, alive: PInteger): integer;
  cdecl; external LIBQ3H;
function q3h_frame_state(f: q3h_frame; stream: integer;
  logits, past_hidden: PSingle): integer; cdecl; external LIBQ3H;
function q3h_frame_destroy(f: q3h_frame): integer; cdecl; external LIBQ3H;
function q3h_frame_set_sampling(f: q3h_frame; s: Pq3h_sampling): integer;
  cdecl; external LIBQ3H;

{ the text projection and Start on the device (talker.pas:390-421, 471-593) }
function q3h_text_create(dev: q3h_device; cfg: Pq3h_text_config; emb: pointer;
  fc1_w, fc1_b, fc2_w, fc2_b: PSingle; out t: q3h_text_proj): integer;
  cdecl; external LIBQ3H;
function q3h_text_project(t: q3h_text_proj; ids: PInteger; n: integer;
  y: PSingle): integer; cdecl; external LIBQ3H;
function q3h_text_destroy(t: q3h_text_proj): integer; cdecl; external LIBQ3H;
function q3h_frame_start_text(f: q3h_frame; stream: integer; t: q3h_text_proj;
  sp: Pq3h_start_ids; ids: PInteger; n_ids: integer; codec: PInteger;
  n_codec: integer; non_streaming: integer): integer; cdecl; external LIBQ3H;

{ the decoder's back part: TQwenCodecVulkan (codec.vulkan.pas:568-652) }
function q3h_codec_create(dev: q3h_device; w: Pq3h_codec_weights;
  max_frames: integer; out c: q3h_codec): integer; cdecl; external LIBQ3H;
function q3h_codec_reset(c: q3h_codec): integer; cdecl; external LIBQ3H;
function q3h_codec_back(c: q3h_codec; x: PSingle; frames: integer;
  pcm: PSingle): integer; cdecl; external LIBQ3H;
function q3h_codec_bytes(c: q3h_codec): Int64; cdecl; external LIBQ3H;
function q3h_codec_destroy(c: q3h_codec): integer; cdecl; external LIBQ3H;

{ helpers }
function q3h_quantize_row_q8_0(x: PSingle; y: pointer; k: Int64): integer;
  cdecl; external LIBQ3H;
function q3h_stack_time_gemv(s: q3h_stack; head, iters, mode: integer;
  out us_per_launch: single; out launches: integer; out bytes: Int64): integer;
  cdecl; external LIBQ3H;

type
  /// what the library reports, with its message (EQwenLm for lm.pas callers)
  EQwenHip = class(Exception);

  TQwen3HipContext = class;

  /// the device-resident layers of one Qwen3 stack, as TQwen3Vulkan holds
  // them (lm.pas:351): the weights go to the device at the first NewContext
  // (after KvF16 is set, as lm.pas:352-353 orders it), then the host weights
  // may be freed
  TQwen3Hip = class
  protected
    fDevice: q3h_device;
    fConfig: q3h_stack_config;
    fWeights: q3h_weights;
    fStack: q3h_stack;
    procedure SetKvF16(aValue: boolean);
    function GetKvF16: boolean;
  public
    /// aWeights^.layers and the arrays it points to must live until the
    // first NewContext
    constructor Create(aDevice: q3h_device; const aConfig: q3h_stack_config;
      const aWeights: q3h_weights);
    destructor Destroy; override;
    /// TQwenLmHeads.Add (lm.pas:277-308): a head [aRows][hidden] in
    // aSrcDType, returned index = the aOutput of ForwardEmbeds
    function AddHead(aRows: pointer; aRowCount, aSrcDType: integer): integer;
    /// a new context of up to aMaxPositions positions (lm.pas:353)
    function NewContext(aMaxPositions: integer): TQwen3HipContext;
    property KvF16: boolean read GetKvF16 write SetKvF16;
    property Stack: q3h_stack read fStack;
  end;

  /// one K/V cache of a TQwen3Hip stack (TDecoderContext)
  TQwen3HipContext = class
  protected
    fCtx: q3h_context;
  public
    destructor Destroy; override;
    /// lm.pas:377: the next row is at position 0
    procedure Reset;
    /// ForwardEmbeds(ctx, x, rows, nil, false, aNormed) and the head product
    // of lm.pas:397-406 in one call: aHead -1 for no logits
    procedure ForwardEmbeds(x: PSingle; aRows, aHead: integer;
      aLogits, aNormed: PSingle);
    function Length: integer;
    property Handle: q3h_context read fCtx;
  end;

/// raise EQwenHip with the library message when rc <> Q3H_OK
procedure Q3hCheck(rc: integer; const what: string);


implementation

procedure Q3hCheck(rc: integer; const what: string);
begin
  if rc <> Q3H_OK then
    raise EQwenHip.CreateFmt('%s: q3h error %d: %s',
      [what, rc, string(AnsiString(q3h_last_error))]);
end;


{ TQwen3Hip }

constructor TQwen3Hip.Create(aDevice: q3h_device; const aConfig: q3h_stack_config;
  const aWeights: q3h_weights);
begin
  inherited Create;
  fDevice := aDevice;
  fConfig := aConfig;
  fWeights := aWeights;
end;

destructor TQwen3Hip.Destroy;
begin
  if fStack <> nil then
    q3h_stack_destroy(fStack); // its contexts are destroyed first (lm.pas:364-368)
  inherited Destroy;
end;

procedure TQwen3Hip.SetKvF16(aValue: boolean);
begin
  if fStack <> nil then
    raise EQwenHip.Create('TQwen3Hip.KvF16: set it before the first NewContext');
  fConfig.kv_f16 := ord(aValue);
end;

function TQwen3Hip.GetKvF16: boolean;
begin
  result := fConfig.kv_f16 <> 0;
end;

function TQwen3Hip.AddHead(aRows: pointer; aRowCount, aSrcDType: integer): integer;
begin
  if fStack = nil then
    Q3hCheck(q3h_stack_create(fDevice, @fConfig, @fWeights, fStack), 'q3h_stack_create');
  Q3hCheck(q3h_stack_add_head(fStack, aRows, aRowCount, aSrcDType, result),
    'q3h_stack_add_head');
end;

function TQwen3Hip.NewContext(aMaxPositions: integer): TQwen3HipContext;
var
  c: q3h_context;
begin
  if fStack = nil then
    Q3hCheck(q3h_stack_create(fDevice, @fConfig, @fWeights, fStack), 'q3h_stack_create');
  Q3hCheck(q3h_context_create(fStack, aMaxPositions, c), 'q3h_context_create');
  result := TQwen3HipContext.Create;
  result.fCtx := c;
end;


{ TQwen3HipContext }

destructor TQwen3HipContext.Destroy;
begin
  if fCtx <> nil then
    q3h_context_destroy(fCtx);
  inherited Destroy;
end;

procedure TQwen3HipContext.Reset;
begin
  Q3hCheck(q3h_context_reset(fCtx), 'q3h_context_reset');
end;

procedure TQwen3HipContext.ForwardEmbeds(x: PSingle; aRows, aHead: integer;
  aLogits, aNormed: PSingle);
begin
  Q3hCheck(q3h_forward_embeds(fCtx, x, aRows, aHead, aLogits, aNormed),
    'q3h_forward_embeds');
end;

function TQwen3HipContext.Length: integer;
begin
  result := q3h_context_length(fCtx);
  if result < 0 then
    Q3hCheck(result, 'q3h_context_length');
end;

end.
